// Dense generators wider than 16 channels (16 < d <= 32), depths 1 and 2, on MI355X (gfx950): the series leaf and
// the Van Loan leaf with their flows, the Chen scan and the custom-VJP backward, behind the ews_dense_* entry points.
//
// Reference path (sign convention of the reference: the flow over a clock step h is M = expm_scheme(-h A)):
//   series leaf   ews/core/series_leaf.py:72-126 (letters b_0 = v, b_p = (-h/p) A b_{p-1}; level 1
//                 sum_p b_p / (p + 1), level 2 sum_{p+r<=q} b_p (x) b_r / ((p + r + 2)(r + 1)))
//   Van Loan leaf ews/core/van_loan.py:31-184 (knots of the augmented exponential, reweighted by W = C^{-M}) and
//                 the knot signature of ews/core/signature.py:20-35
//   schemes       ews/core/expm_approx.py:13-41 (exact, euler, cayley, [2/2] pade)
//   flows         ews/core/chen_scan.py:155-168 (per interval, or one shared step)
//   Chen combine  ews/core/chen_scan.py:98-214 and the dense kernel ews/core/kernels/pallas_combine.py:803-858
//   adjoints      the custom VJP of the dense kernel (pallas_combine.py:2360-2565) and JAX autodiff through the
//                 leaf and the scheme of each matrix function
//
// Every matrix is padded to 32 x 32 and every vector to 32 entries with zeros (the padded block of a flow is the
// identity, which maps the zero padding of the states to zero). A workgroup of 256 threads works on one 32 x 32
// matrix at a time in LDS (row pitch 36, so the 8 rows a wavefront touches sit on distinct banks): thread t owns
// row t / 8, columns 4 (t % 8) .. +3 of every product; matrix-vector products reduce over the 8 lanes of a row.
//
// Passes of the forward (per sample b, intervals t = 0 .. n-1, chunks of T intervals):
//   k_wmat    the step matrices: the flow F = scheme(-c A) and the Van Loan pair (P, V) of a = c A, per interval or
//             once per sample (uniform modes). exp / phi: Taylor polynomial of degree 12 on X / 2^s (||.||_1 <= 1),
//             then s doublings (e^{2Y} = (e^Y)^2, phi(2Y) = phi(Y)(I + e^Y)/2); rational schemes: Gauss-Jordan
//             elimination with partial pivoting.
//   k_wleaf   the local terms (s1, s2) of each interval.
//   k_wscan   SUMMARY: each chunk from the zero state, its summary and flow product; ROWS: each chunk from its
//             carry, the rows.
//   k_wcarry  one workgroup per sample: the carries (state before each chunk) from the summaries.
// The Chen step (chen_scan.py:98-152): S1' = F S1 + s1, S2' = F S2 F^T + (F S1) s1^T + s2.
//
// Backward: the row cotangents g_t (readout adjoint), then with lambda the cotangent of the state after a step
//   lambda_{t-1} = g_{t-1} + R_t^T lambda_t:  lambda1 <- F^T (lambda1 + lambda2 s1),  lambda2 <- F^T lambda2 F,
//   ds1 = lambda1 + lambda2^T (F S1),  ds2 = lambda2,
//   dF = (lambda1 + lambda2 s1) S1^T + lambda2 F S2^T + lambda2^T F S2   (S: the state before the step),
// chunk-parallel: each chunk's own part from a zero cotangent at its end (k_wadj LOCAL), a reverse scan of the
// chunks' transposed Chen maps (k_wadj_carry), then each chunk from its end cotangent (k_wadj FULL). Then the
// leaf adjoints (k_wleaf_bwd) and the matrix functions' adjoints (k_wmat_bwd): for the rational schemes through
// d(N^{-1}) = -N^{-1} dN N^{-1}; for exact exp and phi through the block identity
//   f([[Z^T, G], [0, Z^T]]) = [[f(Z^T), L_f(Z^T)[G]], [0, f(Z^T)]],  L_f(Z)^*[G] = L_f(Z^T)[G],
// on a 64 x 64 block matrix (G scaled to the norm of Z, the result scaled back). dA is summed over workgroup
// partials in float64 in a fixed order.
#include <hip/hip_runtime.h>

#include <math.h>

#include <algorithm>
#include <climits>
#include <type_traits>

#include "ews_hip.h"
#include "ews_lanes.h"
#include "ews_wide.h"

namespace ews {
namespace wide {
using lanes::colsum8;
using lanes::sum64;
using lanes::sum8;

constexpr int DP = 32;            // padded channels
constexpr int MM = DP * DP;       // floats of a padded matrix in global memory (row-major, pitch 32)
constexpr int RW = DP + MM;       // floats of a padded state / local-term row (level 1, then level 2)
constexpr int NT = 256;           // threads of every workgroup
constexpr int VMAXK = 64;         // Van Loan knots per interval at most
constexpr int QMAXW = 40;         // series order at most

template <int NM>
struct Geo {
  static constexpr int P = NM + 4;         // LDS row pitch
  static constexpr int SZ = NM * P;        // floats of one LDS matrix
  static constexpr int TPR = NT / NM;      // threads per row
  static constexpr int CPT = NM / TPR;     // columns per thread
};
constexpr int P32 = Geo<32>::P, S32 = Geo<32>::SZ;

template <int NM>
__device__ __forceinline__ int trow() { return (int)threadIdx.x / Geo<NM>::TPR; }
template <int NM>
__device__ __forceinline__ int tcol() { return ((int)threadIdx.x % Geo<NM>::TPR) * Geo<NM>::CPT; }

// acc[c] = sum_k X(i, k) Y(k, j0 + c) for the thread's row i and columns j0 ..; X(i, k) = X[k][i] when TX, and
// Y(k, j) = Y[j][k] when TY (S: float or double)
template <int NM, bool TX, bool TY, typename S>
__device__ __forceinline__ void mm(const S* X, const S* Y, S* acc) {
  constexpr int P = Geo<NM>::P, CPT = Geo<NM>::CPT;
  const int i = trow<NM>(), j0 = tcol<NM>();
#pragma unroll
  for (int c = 0; c < CPT; ++c) acc[c] = S(0);
#pragma unroll 4
  for (int k = 0; k < NM; ++k) {
    const S x = TX ? X[k * P + i] : X[i * P + k];
    if constexpr (!TY && std::is_same<S, float>::value) {
#pragma unroll
      for (int c = 0; c < CPT; c += 4) {
        const float4 y = *reinterpret_cast<const float4*>(Y + k * P + j0 + c);
        acc[c] = fmaf(x, y.x, acc[c]);
        acc[c + 1] = fmaf(x, y.y, acc[c + 1]);
        acc[c + 2] = fmaf(x, y.z, acc[c + 2]);
        acc[c + 3] = fmaf(x, y.w, acc[c + 3]);
      }
    } else {
#pragma unroll
      for (int c = 0; c < CPT; ++c) acc[c] = fma(x, TY ? Y[(j0 + c) * P + k] : Y[k * P + j0 + c], acc[c]);
    }
  }
}

template <int NM, typename S>
__device__ __forceinline__ void st(S* Z, const S* acc) {
  constexpr int P = Geo<NM>::P, CPT = Geo<NM>::CPT;
  const int i = trow<NM>(), j0 = tcol<NM>();
#pragma unroll
  for (int c = 0; c < CPT; ++c) Z[i * P + j0 + c] = acc[c];
}

template <int NM, typename S>
__device__ __forceinline__ void ld(const S* Z, S* acc) {
  constexpr int P = Geo<NM>::P, CPT = Geo<NM>::CPT;
  const int i = trow<NM>(), j0 = tcol<NM>();
#pragma unroll
  for (int c = 0; c < CPT; ++c) acc[c] = Z[i * P + j0 + c];
}

// the thread's four entries of a padded 32 x 32 matrix in global memory (pitch 32)
__device__ __forceinline__ float4 gld4(const float* g) {
  return *reinterpret_cast<const float4*>(g + trow<32>() * DP + tcol<32>());
}
__device__ __forceinline__ void gst4(float* g, float4 v) {
  *reinterpret_cast<float4*>(g + trow<32>() * DP + tcol<32>()) = v;
}
__device__ __forceinline__ void sld4(float* Z, float4 v) {
  *reinterpret_cast<float4*>(Z + trow<32>() * P32 + tcol<32>()) = v;
}
__device__ __forceinline__ float4 lds4(const float* Z) {
  return *reinterpret_cast<const float4*>(Z + trow<32>() * P32 + tcol<32>());
}
__device__ __forceinline__ float4 f4add(float4 a, float4 b) {
  return float4{a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w};
}
__device__ __forceinline__ float4 acc4(const float* a) { return float4{a[0], a[1], a[2], a[3]}; }

// y[i] = sum_k M(i, k) x[k] (M(i, k) = M[k][i] when TM), 32 x 32 in LDS: the 8 lanes of row i each take four k and
// sum them (a DPP sum over the 8 lanes); every lane of the row returns y[i]
template <bool TM>
__device__ __forceinline__ float mv(const float* M, const float* x) {
  const int i = (int)threadIdx.x >> 3, p = ((int)threadIdx.x & 7) * 4;
  float s = 0.0f;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int k = p + r;
    s = fmaf(TM ? M[k * P32 + i] : M[i * P32 + k], x[k], s);
  }
  return sum8(s);
}
__device__ __forceinline__ bool row_lead() { return (threadIdx.x & 7) == 0; }

// 32 x 32 products of the scans on fp32 MFMA (mfma_f32_16x16x4f32): wavefront w computes the 16 x 16 tile
// (rows m0 = 16 (w / 2), columns n0 = 16 (w % 2)) of Z = X Y (X(m, k) = X[k][m] when TX, Y(k, n) = Y[n][k] when TY),
// LDS operands at pitch 36; lane (i, g) gives A[m0 + i][k] and B[k][n0 + i] for k = 4u + g and holds the result rows
// m0 + 4g + r (r = 0..3) of column n0 + i.
typedef float v4f __attribute__((ext_vector_type(4)));
__device__ __forceinline__ int tile_m0() { return 16 * ((int)threadIdx.x >> 7); }
__device__ __forceinline__ int tile_n0() { return 16 * (((int)threadIdx.x >> 6) & 1); }
__device__ __forceinline__ int tile_i() { return (int)threadIdx.x & 15; }
__device__ __forceinline__ int tile_g() { return ((int)threadIdx.x >> 4) & 3; }

template <bool TX, bool TY>
__device__ __forceinline__ v4f mm_tile(const float* X, const float* Y, v4f acc, int ku = 8) {
  const int m0 = tile_m0(), n0 = tile_n0(), i = tile_i(), g = tile_g();
#pragma unroll
  for (int u = 0; u < 8; ++u) {
    if (u < ku) {  // (uniform) the k-steps past ku read only zero padding of one factor
      const int k = 4 * u + g;
      const float xa = TX ? X[k * P32 + m0 + i] : X[(m0 + i) * P32 + k];
      const float yb = TY ? Y[(n0 + i) * P32 + k] : Y[k * P32 + n0 + i];
      acc = __builtin_amdgcn_mfma_f32_16x16x4f32(xa, yb, acc, 0, 0, 0);
    }
  }
  return acc;
}
__device__ __forceinline__ v4f zero4() { return v4f{0.0f, 0.0f, 0.0f, 0.0f}; }
// float64 products on MFMA (mfma_f64_16x16x4f64): the wavefront's 16 x 16 tile of Z = X Y (X(m, k) = X[k][m] when
// TX, Y(k, n) = Y[n][k] when TY), LDS at pitch 36. The operands are laid out as for mfma_f32_16x16x4f32 (lane
// (i, g): X(m0 + i, 4 u + g), Y(4 u + g, n0 + i)), but the result rows are interleaved: lane (i, g) holds rows
// m0 + g + 4 r (r = 0..3) of column n0 + i (a probe with one-hot operands showed it)
typedef double v4d __attribute__((ext_vector_type(4)));
template <bool TX, bool TY>
__device__ __forceinline__ v4d mm_tile_d(const double* X, const double* Y, v4d acc) {
  const int m0 = tile_m0(), n0 = tile_n0(), i = tile_i(), g = tile_g();
#pragma unroll
  for (int u = 0; u < 8; ++u) {
    const int k = 4 * u + g;
    const double xa = TX ? X[k * P32 + m0 + i] : X[(m0 + i) * P32 + k];
    const double yb = TY ? Y[(n0 + i) * P32 + k] : Y[k * P32 + n0 + i];
    acc = __builtin_amdgcn_mfma_f64_16x16x4f64(xa, yb, acc, 0, 0, 0);
  }
  return acc;
}
__device__ __forceinline__ int tile_row_d(int r) { return tile_m0() + tile_g() + 4 * r; }  // result row of item r
__device__ __forceinline__ void st_tile_d(double* Z, v4d v) {
  const int n = tile_n0() + tile_i();
#pragma unroll
  for (int r = 0; r < 4; ++r) Z[tile_row_d(r) * P32 + n] = v[r];
}
// the lane's tile entries of a 32 x 32 matrix: LDS (pitch 36) or global (pitch 32)
__device__ __forceinline__ void st_tile(float* Z, v4f v) {
  const int m = tile_m0() + 4 * tile_g(), n = tile_n0() + tile_i();
#pragma unroll
  for (int r = 0; r < 4; ++r) Z[(m + r) * P32 + n] = v[r];
}
__device__ __forceinline__ v4f gld_tile(const float* g) {
  const int m = tile_m0() + 4 * tile_g(), n = tile_n0() + tile_i();
  return v4f{g[m * DP + n], g[(m + 1) * DP + n], g[(m + 2) * DP + n], g[(m + 3) * DP + n]};
}
__device__ __forceinline__ void gst_tile(float* g, v4f v) {
  const int m = tile_m0() + 4 * tile_g(), n = tile_n0() + tile_i();
#pragma unroll
  for (int r = 0; r < 4; ++r) g[(m + r) * DP + n] = v[r];
}

// sum over the workgroup (every thread returns it); red: NT / 64 floats of LDS
__device__ __forceinline__ float block_sum(float v, float* red) {
  v = sum64(v);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  float s = 0.0f;
#pragma unroll
  for (int w = 0; w < NT / 64; ++w) s += red[w];
  return s;
}

// ------------------------------------------------------------------------------------------------ matrix functions
// The forward's step matrices are formed in float64 (S = double; each is reused at every step of its sample, so its
// rounding would add up along the scan) and stored in float32; the adjoints run in float32 (S = float).

// ||X||_1 (largest column sum of magnitudes), NM x NM in LDS; every thread returns it. red: NM entries.
template <int NM, typename S>
__device__ S norm1(const S* X, S* red) {
  constexpr int P = Geo<NM>::P;
  __syncthreads();
  if ((int)threadIdx.x < NM) {
    S s = S(0);
    for (int r = 0; r < NM; ++r) s += fabs(X[r * P + threadIdx.x]);
    red[threadIdx.x] = s;
  }
  __syncthreads();
  S m = S(0);
  for (int c = 0; c < NM; ++c) m = fmax(m, red[c]);
  __syncthreads();
  return m;
}

// E = exp(X), Ph = phi(X) = sum_k X^k / (k + 1)! (NM x NM in LDS; X is overwritten with X / 2^s). Taylor polynomial of
// degree 12 of phi in Y = X / 2^s with ||Y||_1 <= 1 (remainder below 1/13!), E = I + Y phi(Y), then s doublings
// phi(2Y) = phi(Y)(I + e^Y)/2, e^{2Y} = e^Y e^Y. T1, T2: scratch matrices; red: NM entries.
template <int NM, typename S>
__device__ void exp_phi(S* X, S* E, S* Ph, S* T1, S* T2, S* red) {
  constexpr int CPT = Geo<NM>::CPT;
  const int i = trow<NM>(), j0 = tcol<NM>();
  const S nrm = norm1<NM>(X, red);
  int s = 0;
  S sc = S(1);
  while (nrm * sc > S(1) && s < 64) {
    sc *= S(0.5);
    ++s;
  }
  S acc[CPT];
  ld<NM>(X, acc);
#pragma unroll
  for (int c = 0; c < CPT; ++c) acc[c] *= sc;
  __syncthreads();
  st<NM>(X, acc);
  // Horner: R = c_12 I, R <- c_k I + Y R (k = 11 .. 0), c_k = 1 / (k + 1)!
  S ck = S(1);
  for (int k = 1; k <= 13; ++k) ck /= S(k);  // 1 / 13!
#pragma unroll
  for (int c = 0; c < CPT; ++c) acc[c] = (i == j0 + c) ? ck : S(0);
  st<NM>(T1, acc);
  __syncthreads();
  S* R = T1;
  S* Rn = T2;
  for (int k = 11; k >= 0; --k) {
    ck *= S(k + 2);  // 1 / (k + 1)!
    mm<NM, false, false>(X, R, acc);
#pragma unroll
    for (int c = 0; c < CPT; ++c) acc[c] += (i == j0 + c) ? ck : S(0);
    st<NM>(Rn, acc);
    __syncthreads();
    S* tmp = R;
    R = Rn;
    Rn = tmp;
  }
  mm<NM, false, false>(X, R, acc);
#pragma unroll
  for (int c = 0; c < CPT; ++c) acc[c] += (i == j0 + c) ? S(1) : S(0);
  st<NM>(E, acc);
  S ph[CPT];
  ld<NM>(R, ph);
  st<NM>(Ph, ph);
  __syncthreads();
  for (int r = 0; r < s; ++r) {
    S pe[CPT];
    mm<NM, false, false>(Ph, E, pe);
    mm<NM, false, false>(E, E, acc);
    __syncthreads();
#pragma unroll
    for (int c = 0; c < CPT; ++c) ph[c] = S(0.5) * (ph[c] + pe[c]);
    st<NM>(Ph, ph);
    st<NM>(E, acc);
    __syncthreads();
  }
}

// Y = N^{-1} (32 x 32 in LDS) by Gauss-Jordan elimination on [N | I] with partial pivoting (largest magnitude in the
// column among the rows not yet reduced, ties to the lower row; rows are swapped). Aug: 32 x 68 entries of LDS;
// sh: 64 entries of LDS.
template <typename S>
__device__ void inv32(const S* Nm, S* Y, S* Aug, S* sh) {
  constexpr int AP = 68;
  const int tid = threadIdx.x;
  for (int e = tid; e < 32 * 64; e += NT) {
    const int r = e >> 6, c = e & 63;
    Aug[r * AP + c] = c < 32 ? Nm[r * P32 + c] : (c - 32 == r ? S(1) : S(0));
  }
  __syncthreads();
  for (int k = 0; k < 32; ++k) {
    if (tid < 64) {  // wavefront 0: the pivot row
      S v = (tid < 32 && tid >= k) ? fabs(Aug[tid * AP + k]) : S(-1);
      int r = tid;
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) {
        const S v2 = __shfl_xor(v, o, 64);
        const int r2 = __shfl_xor(r, o, 64);
        if (v2 > v || (v2 == v && r2 < r)) {
          v = v2;
          r = r2;
        }
      }
      if (tid == 0) sh[32] = S(r);
    }
    __syncthreads();
    const int pr = (int)sh[32];
    if (pr != k && tid < 64) {
      const S a = Aug[k * AP + tid], b = Aug[pr * AP + tid];
      Aug[k * AP + tid] = b;
      Aug[pr * AP + tid] = a;
    }
    __syncthreads();
    if (tid < 32) sh[tid] = Aug[tid * AP + k];  // the elimination factors (column k)
    __syncthreads();
    const S inv = S(1) / sh[k];
    if (tid < 64) Aug[k * AP + tid] *= inv;
    __syncthreads();
    for (int e = tid; e < 32 * 64; e += NT) {
      const int r = e >> 6, c = e & 63;
      if (r != k) Aug[r * AP + c] = fma(-sh[r], Aug[k * AP + c], Aug[r * AP + c]);
    }
    __syncthreads();
  }
  for (int e = tid; e < 32 * 32; e += NT) {
    const int r = e >> 5, c = e & 31;
    Y[r * P32 + c] = Aug[r * AP + 32 + c];
  }
  __syncthreads();
}

// LDS layout of the matrix-function workgroups (entries of S): A, X, Y, T, U, N (32 x 36 each), Aug (32 x 68), small;
// then the exact scheme's block area: five 32 x 36 matrices in the forward, five 64 x 68 in the adjoint.
constexpr int MF_A = 0, MF_X = S32, MF_Y = 2 * S32, MF_T = 3 * S32, MF_U = 4 * S32, MF_N = 5 * S32;
constexpr int MF_AUG = 6 * S32, MF_SH = MF_AUG + 32 * 68, MF_RED = MF_SH + 64, MF_BLK = MF_RED + 64;
constexpr int S64 = Geo<64>::SZ;
constexpr int MF_ENT_FWD = MF_BLK + 5 * S32, MF_ENT_BWD = MF_BLK, MF_ENT_BWD_EXACT = MF_BLK + 5 * S64;

template <typename S>
__device__ __forceinline__ void set_ident32(S* Z, S diag) {
  const int i = trow<32>(), j0 = tcol<32>();
  S a[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) a[c] = (i == j0 + c) ? diag : S(0);
  st<32>(Z, a);
}

// N = I + alpha X + beta X^2 into U (X in LDS)
template <typename S>
__device__ void form_n(const S* X, S* U, S alpha, S beta) {
  const int i = trow<32>(), j0 = tcol<32>();
  S x2[4] = {S(0), S(0), S(0), S(0)}, x[4];
  if (beta != S(0)) mm<32, false, false>(X, X, x2);
  ld<32>(X, x);
  S n[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) n[c] = ((i == j0 + c) ? S(1) : S(0)) + alpha * x[c] + beta * x2[c];
  st<32>(U, n);
  __syncthreads();
}

__device__ __forceinline__ void scheme_ab(int scheme, bool flow, double& alpha, double& beta) {
  // N = I + alpha X + beta X^2 of the rational schemes (the flow's cayley / pade, the Van Loan V)
  alpha = 0.5;
  beta = 0.0;
  if (scheme == EWS_EXPM_PADE) beta = 1.0 / 12.0;
  if (scheme == EWS_EXPM_EULER && !flow) alpha = 1.0;
}

template <typename S>
__device__ __forceinline__ void load_A(int d, const float* Ag, S* A) {
  for (int e = threadIdx.x; e < MM; e += NT) {
    const int r = e >> 5, c = e & 31;
    A[r * P32 + c] = (r < d && c < d) ? S(Ag[r * d + c]) : S(0);
  }
}

// Forward matrix functions of X = c A in float64 (A, X in the LDS layout above): flow F = scheme(-X) into out0, or
// the Van Loan pair P into out0, V into out1 (global float32, pitch 32).
__device__ void matfn_fwd(double* sm, int scheme, bool flow, double c, float* out0, float* out1) {
  double* A = sm + MF_A;
  double* X = sm + MF_X;
  double* Y = sm + MF_Y;
  double* U = sm + MF_U;
  const int i = trow<32>(), j0 = tcol<32>();
  double a[4];
  ld<32>(A, a);
#pragma unroll
  for (int k = 0; k < 4; ++k) a[k] *= c;
  st<32>(X, a);
  __syncthreads();
  double r0[4], r1[4];
  if (scheme == EWS_EXPM_EXACT) {
    double* B = sm + MF_BLK;  // Z = -X, E = exp(Z), Ph = phi(Z)
    double* Z = B;
    double* E = B + S32;
    double* Ph = B + 2 * S32;
#pragma unroll
    for (int k = 0; k < 4; ++k) a[k] = -a[k];
    st<32>(Z, a);
    __syncthreads();
    exp_phi<32>(Z, E, Ph, B + 3 * S32, B + 4 * S32, sm + MF_RED);
    ld<32>(E, r0);
    ld<32>(Ph, r1);
  } else if (flow && scheme == EWS_EXPM_EULER) {
#pragma unroll
    for (int k = 0; k < 4; ++k) r0[k] = ((i == j0 + k) ? 1.0 : 0.0) - a[k];
  } else {
    double alpha, beta;
    scheme_ab(scheme, flow, alpha, beta);
    form_n(X, U, alpha, beta);
    inv32(U, Y, sm + MF_AUG, sm + MF_SH);
    double y[4];
    ld<32>(Y, y);
    if (scheme == EWS_EXPM_PADE) {  // F = I - Y X (flow), P = I - V X (Van Loan, V = Y)
      double yx[4];
      mm<32, false, false>(Y, X, yx);
#pragma unroll
      for (int k = 0; k < 4; ++k) r0[k] = ((i == j0 + k) ? 1.0 : 0.0) - yx[k];
    } else if (scheme == EWS_EXPM_CAYLEY) {  // F = P = 2Y - I
#pragma unroll
      for (int k = 0; k < 4; ++k) r0[k] = 2.0 * y[k] - ((i == j0 + k) ? 1.0 : 0.0);
    } else {  // Van Loan euler: P = V = Y
#pragma unroll
      for (int k = 0; k < 4; ++k) r0[k] = y[k];
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) r1[k] = y[k];
  }
  gst4(out0, float4{(float)r0[0], (float)r0[1], (float)r0[2], (float)r0[3]});
  if (!flow) gst4(out1, float4{(float)r1[0], (float)r1[1], (float)r1[2], (float)r1[3]});
  __syncthreads();
}

// Adjoint of matfn_fwd (float32): given the cotangents G0 (of F, or of P) and G1 (of V; unused for a flow) in LDS
// (T, U), returns in xb the thread's four entries of the cotangent of X = c A.
__device__ void matfn_bwd(float* sm, int scheme, bool flow, float c, float* xb) {
  float* A = sm + MF_A;
  float* X = sm + MF_X;
  float* Y = sm + MF_Y;
  float* G0 = sm + MF_T;
  float* G1 = sm + MF_U;
  const int i = trow<32>(), j0 = tcol<32>();
  float a[4];
  ld<32>(A, a);
#pragma unroll
  for (int k = 0; k < 4; ++k) a[k] *= c;
  st<32>(X, a);
  __syncthreads();
  if (scheme == EWS_EXPM_EXACT) {
    // Z = -X; dZ = L_exp(Z^T)[G0] (+ L_phi(Z^T)[G1]); each from the 64 x 64 block [[Z^T, G/tau], [0, Z^T]]
    float* B = sm + MF_BLK;
    constexpr int P = Geo<64>::P;
    const float zn = fmaxf(norm1<32>(X, sm + MF_RED), 1.0f);  // G is scaled to at most max(||Z||_1, 1)
    float dz[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int pass = 0; pass < (flow ? 1 : 2); ++pass) {
      const float* Gs = pass == 0 ? G0 : G1;
      const float gn = norm1<32>(Gs, sm + MF_RED);
      if (gn == 0.0f) continue;  // uniform over the workgroup
      const float tau = gn / zn;
      for (int e = threadIdx.x; e < 64 * 64; e += NT) {
        const int r = e >> 6, q = e & 63;
        float v = 0.0f;
        if (r < 32 && q < 32) v = -X[q * P32 + r];                   // Z^T
        else if (r >= 32 && q >= 32) v = -X[(q - 32) * P32 + (r - 32)];
        else if (r < 32 && q >= 32) v = Gs[r * P32 + (q - 32)] / tau;
        B[r * P + q] = v;
      }
      __syncthreads();
      exp_phi<64>(B, B + S64, B + 2 * S64, B + 3 * S64, B + 4 * S64, sm + MF_RED);
      const float* R = pass == 0 ? B + S64 : B + 2 * S64;  // exp for P (or F), phi for V
#pragma unroll
      for (int k = 0; k < 4; ++k) dz[k] = fmaf(tau, R[i * P + 32 + j0 + k], dz[k]);
      __syncthreads();
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) xb[k] = -dz[k];
    return;
  }
  float g0[4];
  ld<32>(G0, g0);
  if (flow && scheme == EWS_EXPM_EULER) {  // F = I - X
#pragma unroll
    for (int k = 0; k < 4; ++k) xb[k] = -g0[k];
    return;
  }
  double alpha_d, beta_d;
  scheme_ab(scheme, flow, alpha_d, beta_d);
  const float alpha = (float)alpha_d, beta = (float)beta_d;
  form_n(X, sm + MF_N, alpha, beta);
  inv32(sm + MF_N, Y, sm + MF_AUG, sm + MF_SH);
  // Yb: the cotangent of Y; direct: the part of dX not through Y
  float yb[4], direct[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  if (scheme == EWS_EXPM_PADE) {
    float t[4];
    mm<32, false, true>(G0, X, t);       // G0 X^T
    mm<32, true, false>(Y, G0, direct);  // Y^T G0
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      yb[k] = -t[k];
      direct[k] = -direct[k];
    }
  } else if (scheme == EWS_EXPM_CAYLEY) {
#pragma unroll
    for (int k = 0; k < 4; ++k) yb[k] = 2.0f * g0[k];
  } else {  // Van Loan euler: P = V = Y
#pragma unroll
    for (int k = 0; k < 4; ++k) yb[k] = g0[k];
  }
  if (!flow) {
    float g1[4];
    ld<32>(G1, g1);
#pragma unroll
    for (int k = 0; k < 4; ++k) yb[k] += g1[k];
  }
  // Nb = -Y^T Yb Y^T;  dX = direct + alpha Nb + beta (Nb X^T + X^T Nb)
  float* W1 = sm + MF_AUG;  // free after the inverse (32 x 68 >= 32 x 36)
  __syncthreads();
  st<32>(W1, yb);
  __syncthreads();
  float t1[4];
  mm<32, false, true>(W1, Y, t1);  // Yb Y^T
  __syncthreads();
  st<32>(W1, t1);
  __syncthreads();
  float nb[4];
  mm<32, true, false>(Y, W1, nb);  // Y^T (Yb Y^T)
#pragma unroll
  for (int k = 0; k < 4; ++k) nb[k] = -nb[k];
  __syncthreads();
  st<32>(W1, nb);
  __syncthreads();
#pragma unroll
  for (int k = 0; k < 4; ++k) xb[k] = direct[k] + alpha * nb[k];
  if (beta != 0.0f) {
    float p1[4], p2[4];
    mm<32, false, true>(W1, X, p1);  // Nb X^T
    mm<32, true, false>(X, W1, p2);  // X^T Nb
#pragma unroll
    for (int k = 0; k < 4; ++k) xb[k] = fmaf(beta, p1[k] + p2[k], xb[k]);
  }
  __syncthreads();
}

// ------------------------------------------------------------------------------------------------ steps
// Clock step of the flow of interval t (chen_scan.py:155-168): per interval, or the shared step; interval 0 of the
// basepoint mode has the identity flow.
__device__ __forceinline__ float flow_step(const WArgs& a, const float* th, int t, bool& ident) {
  ident = false;
  if (a.flow_mode == EWS_FLOW_PER_INTERVAL) return th[t + 1] - th[t];
  if (a.flow_mode == EWS_FLOW_CACHED) return th[1] - th[0];
  ident = t == 0;
  return th[2] - th[1];
}
// Van Loan step dt / M of interval t (van_loan.py:31-160): per interval; the uniform modes share dt = th[1] - th[0]
// (or th[2] - th[1] with the pure jump at interval 0 of the basepoint mode); a shared dt <= 1e-12 is the jump
// (linear knots: P = V = I, fixed = true).
__device__ __forceinline__ float vl_step(const WArgs& a, const float* th, int t, bool& fixed) {
  fixed = false;
  if (a.vl_mode == EWS_FLOW_PER_INTERVAL) return (th[t + 1] - th[t]) / (float)a.vm;
  const float dt = a.vl_mode == EWS_FLOW_CACHED ? th[1] - th[0] : th[2] - th[1];
  fixed = !(dt > 1e-12f) || (a.vl_mode == EWS_FLOW_CACHED_BASEPOINT && t == 0);
  return fixed ? 0.0f : dt / (float)a.vm;
}

// The items of a matrix-function workgroup: modes 0 and 1 every gridDim-th item from blockIdx.x; mode 2 (the
// matrices outside the series radius) the flagged items of the workgroup's blocks of NT consecutive intervals
// (blocks blockIdx.x, blockIdx.x + gridDim.x, ...), found by one flag load per thread and a workgroup vote, in
// increasing order. next_item(.., prev) returns the item after prev (prev = -1: the first), or item_end when none
// is left; uniform over the workgroup.
__device__ __forceinline__ long item_end(int mode, long items) { return mode == 2 ? LONG_MAX : items; }
__device__ long next_item(const WArgs& a, int mode, int need, long prev, long items) {
  if (mode != 2) return prev < 0 ? (long)blockIdx.x : prev + gridDim.x;
  __shared__ int s_first;
  long blk = prev < 0 ? (long)blockIdx.x : prev / NT;
  long from = prev < 0 ? blk * NT : prev + 1;
  for (; blk * NT < items; blk += gridDim.x, from = blk * NT) {
    const long it = blk * NT + threadIdx.x;
    const bool f = it >= from && it < items && (a.mflag[it] & need);
    if (threadIdx.x == 0) s_first = NT;
    __syncthreads();
    if (f) atomicMin(&s_first, (int)threadIdx.x);
    __syncthreads();
    const int first = s_first;
    __syncthreads();
    if (first < NT) return blk * NT + first;
  }
  return LONG_MAX;
}

// Step matrices: item = interval (per-interval modes) or sample (shared modes); the flow and the Van Loan pair are
// each formed when their mode matches the item kind.
// mode: 0 per sample, 1 per interval, 2 per interval, only the matrices flagged outside the series radius
__global__ __launch_bounds__(NT) void k_wmat(WArgs a, int mode) {
  extern __shared__ __align__(16) double smd[];
  load_A(a.d, a.A, smd + MF_A);
  __syncthreads();
  const int per_interval = mode != 0;
  const long items = per_interval ? (long)a.B * a.n : a.B;
  // with two grid rows, row 0 forms the flows and row 1 the Van Loan pairs
  const bool do_flow = (a.flow_mode == EWS_FLOW_PER_INTERVAL) == (per_interval != 0) &&
                       (gridDim.y == 1 || blockIdx.y == 0);
  const bool do_vl = a.leaf == EWS_LEAF_VAN_LOAN && (a.vl_mode == EWS_FLOW_PER_INTERVAL) == (per_interval != 0) &&
                     (gridDim.y == 1 || blockIdx.y == 1);
  const int need = (do_flow ? 1 : 0) | (do_vl ? 2 : 0);
  for (long it = next_item(a, mode, need, -1, items), it_end = item_end(mode, items); it < it_end;
       it = next_item(a, mode, need, it, items)) {
    const int b = per_interval ? (int)(it / a.n) : (int)it;
    const int t = per_interval ? (int)(it - (long)b * a.n) : 1;
    const float* th = a.clock + (size_t)b * a.L;
    const int flag = mode == 2 ? a.mflag[it] : a.sflag[it];  // the matrices outside the series radius
    if (do_flow && (flag & 1)) {
      bool ident;
      const float h = flow_step(a, th, t, ident);
      matfn_fwd(smd, a.chen, true, (double)h, a.fl + it * MM, nullptr);
    }
    if (do_vl && (flag & 2)) {
      bool fixed;
      const float c = vl_step(a, th, t, fixed);
      matfn_fwd(smd, fixed ? EWS_EXPM_EULER : a.vl_expm, false, fixed ? 0.0 : (double)c, a.vlm + it * 2 * MM,
                a.vlm + it * 2 * MM + MM);
    }
  }
}

// ------------------------------------------------------------------------------------------------ series path
// Per-interval matrix functions as power series in X = c A over a table of powers A^0 .. A^PW formed once per call:
// out = sum_k gamma_k c^k A^k, entry by entry (each thread keeps its four entries of every power in registers),
// wherever |c| ||A||_1 is inside the scheme's radius (series remainder below about 1e-11); a matrix outside it is
// flagged and formed by k_wmat (mode 2). The adjoint accumulates H_k = sum_items gamma_k c^k dOut and turns it
// into dA once: dA = sum_k sum_{i<k} (A^T)^i H_k (A^T)^{k-1-i}; the step's cotangent is <dOut, d out / dc>.
// gamma_k (kind 0 the flow scheme(-X); kind 1 the Van Loan P, kind 2 its V):
//   exact   F, P: (-1)^k / k!          V: (-1)^k / (k+1)!
//   cayley  F, P: 1, then 2 (-1/2)^k   V: (-1/2)^k                          ((I + X/2)^{-1})
//   euler   F: 1, -1                   P = V: (-1)^k                         ((I + X)^{-1})
//   pade    F, P: 1, then -b_{k-1}     V: b_k, b_0 = 1, b_1 = -1/2, b_k = -(b_{k-1}/2 + b_{k-2}/12)
constexpr int PW = 18;

__device__ void series_gamma(int scheme, int kind, float* g) {
  double b[PW + 1];
  b[0] = 1.0;
  for (int k = 1; k <= PW; ++k) {
    if (scheme == EWS_EXPM_EXACT) b[k] = -b[k - 1] / (double)(kind == 2 ? k + 1 : k);
    else if (scheme == EWS_EXPM_CAYLEY) b[k] = -0.5 * b[k - 1];
    else if (scheme == EWS_EXPM_EULER) b[k] = -b[k - 1];
    else b[k] = -(0.5 * b[k - 1] + (k >= 2 ? b[k - 2] / 12.0 : 0.0));
  }
  for (int k = 0; k <= PW; ++k) g[k] = 0.0f;
  if (scheme == EWS_EXPM_EULER && kind == 0) {
    g[0] = 1.0f;
    g[1] = -1.0f;
  } else if (kind == 2 || scheme == EWS_EXPM_EXACT || (scheme == EWS_EXPM_EULER && kind == 1)) {
    for (int k = 0; k <= PW; ++k) g[k] = (float)b[k];
  } else if (scheme == EWS_EXPM_CAYLEY) {  // F, P = 2V - I
    g[0] = 1.0f;
    for (int k = 1; k <= PW; ++k) g[k] = (float)(2.0 * b[k]);
  } else {  // pade F, P = I - V X
    g[0] = 1.0f;
    for (int k = 1; k <= PW; ++k) g[k] = (float)(-b[k - 1]);
  }
}
__device__ __forceinline__ float series_radius(int scheme, int kind) {
  if (scheme == EWS_EXPM_EXACT) return 1.0f;
  if (scheme == EWS_EXPM_CAYLEY) return 0.5f;
  if (scheme == EWS_EXPM_EULER) return kind == 0 ? 3.0e38f : 0.25f;
  return 0.7f;
}

// Van Loan knots on the series path: knot r (Delta_{r+1}, r = 0 .. M-1) is f_r(X) w with f_{M-1} = V and
// f_{r-1} = P f_r, analytic in X = c A (P and V commute), so Delta_{r+1} = sum_k phi[r][k] c^k (A^k w); the
// coefficients phi are the products of the schemes' scalar series, truncated at order PW, formed once per call.
// The series holds where M |c| ||A||_1 is inside the scheme's radius.
constexpr int PHI_OFF = (PW + 1) * MM + 64;  // offset of phi in apow (M rows of PW + 1)
constexpr int APOW_FLOATS = PHI_OFF + 64 * (PW + 1);

// the knots' coefficients phi[r][k] of the series path: f_{M-1} = V, f_{r-1} = P f_r as truncated series (float64),
// thread k < PW + 1 forming coefficient k of each
__device__ void wpowers_phi(const WArgs& a) {
  __shared__ float s_gp[PW + 1], s_gv[PW + 1];
  __shared__ double s_f[2][PW + 1];
  if (threadIdx.x == 0) {
    series_gamma(a.vl_expm, 1, s_gp);
    series_gamma(a.vl_expm, 2, s_gv);
  }
  __syncthreads();
  const int k = threadIdx.x;
  if (k <= PW) s_f[0][k] = s_gv[k];
  __syncthreads();
  float* phi = a.apow + PHI_OFF;
  int cur = 0;
  for (int r = a.vm - 1; r >= 0; --r) {
    if (k <= PW) {
      phi[r * (PW + 1) + k] = (float)s_f[cur][k];
      double x = 0.0;
      for (int j = 0; j <= k; ++j) x += (double)s_gp[j] * s_f[cur][k - j];
      s_f[cur ^ 1][k] = x;
    }
    __syncthreads();
    cur ^= 1;
  }
}

// the table: A^k (k = 0 .. PW) in float64, stored float, ||A||_1 at apow[(PW + 1) MM] (workgroup 0); with a
// per-interval Van Loan leaf the knots' coefficients phi at apow[PHI_OFF] (workgroup 1)
__global__ __launch_bounds__(NT) void k_wpowers(WArgs a) {
  if (blockIdx.x == 1) {  // a second workgroup (per-interval Van Loan leaf): the knots' coefficients
    wpowers_phi(a);
    return;
  }
  __shared__ __align__(16) double sd[3 * S32 + 64];
  double* A = sd;
  double* T = sd + S32;
  double* Tn = sd + 2 * S32;
  load_A(a.d, a.A, A);
  set_ident32(T, 1.0);
  __syncthreads();
  const int i = trow<32>(), j0 = tcol<32>();
  gst4(a.apow, float4{i == j0 ? 1.0f : 0.0f, i == j0 + 1 ? 1.0f : 0.0f, i == j0 + 2 ? 1.0f : 0.0f,
                      i == j0 + 3 ? 1.0f : 0.0f});
  const int tn = tile_n0() + tile_i();  // the lane's tile entries: rows tile_row_d(r) of column tn
  for (int k = 1; k <= PW; ++k) {
    const v4d acc = mm_tile_d<false, false>(T, A, v4d{0.0, 0.0, 0.0, 0.0});
    st_tile_d(Tn, acc);
#pragma unroll
    for (int r = 0; r < 4; ++r) a.apow[(size_t)k * MM + tile_row_d(r) * DP + tn] = (float)acc[r];
    __syncthreads();
    double* tmp = T;
    T = Tn;
    Tn = tmp;
  }
  const double nrm = norm1<32>(A, sd + 3 * S32);
  if (threadIdx.x == 0) a.apow[(size_t)(PW + 1) * MM] = (float)nrm;
}

// the thread's four entries of every power
__device__ __forceinline__ void load_powers(const WArgs& a, float4* T) {
#pragma unroll
  for (int k = 0; k <= PW; ++k) T[k] = gld4(a.apow + (size_t)k * MM);
}
__device__ __forceinline__ float4 series_eval(const float4* T, const float* g, float c) {
  float4 r = float4{0.0f, 0.0f, 0.0f, 0.0f};
  float ck = 1.0f;
#pragma unroll
  for (int k = 0; k <= PW; ++k) {
    const float w = g[k] * ck;
    r.x = fmaf(w, T[k].x, r.x);
    r.y = fmaf(w, T[k].y, r.y);
    r.z = fmaf(w, T[k].z, r.z);
    r.w = fmaf(w, T[k].w, r.w);
    ck *= c;
  }
  return r;
}

// per-interval flows and Van Loan pairs on the series path; flags the others (bit 0: the flow, bit 1: the Van Loan
// pair outside the series radius; bit 2: the Van Loan knots by the chain, not by their series)
__global__ __launch_bounds__(NT) void k_wmat_series(WArgs a) {
  __shared__ float s_g[3][PW + 1];
  if (threadIdx.x == 0) {
    series_gamma(a.chen, 0, s_g[0]);
    if (a.leaf == EWS_LEAF_VAN_LOAN) {
      series_gamma(a.vl_expm, 1, s_g[1]);
      series_gamma(a.vl_expm, 2, s_g[2]);
    }
  }
  __syncthreads();
  float4 T[PW + 1];
  load_powers(a, T);
  const float nrm = a.apow[(size_t)(PW + 1) * MM];
  const bool do_flow = a.flow_mode == EWS_FLOW_PER_INTERVAL;
  const bool do_vl = a.leaf == EWS_LEAF_VAN_LOAN && a.vl_mode == EWS_FLOW_PER_INTERVAL;
  const float rf = series_radius(a.chen, 0), rv = series_radius(a.vl_expm, 1);
  const long items = (long)a.B * a.n;
  const int i = trow<32>(), j0 = tcol<32>(), s8 = threadIdx.x & 7;
  // the item's clock step and (series-path knots) increment w = v / M, loaded during the item before
  float nh = 0.0f, nw[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  auto fetch = [&](long it) {
    const int b = (int)(it / a.n), t = (int)(it - (long)b * a.n);
    nh = a.clock[(size_t)b * a.L + t + 1] - a.clock[(size_t)b * a.L + t];
    if (do_vl) {
      const float* xp = a.path + ((size_t)b * a.L + t) * a.d;
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int j = min(j0 + u, a.d - 1);  // in bounds; the padded columns are zeroed below
        nw[u] = xp[a.d + j] - xp[j];
      }
    }
  };
  if ((long)blockIdx.x < items) fetch(blockIdx.x);
  for (long it = blockIdx.x; it < items; it += gridDim.x) {
    const float h = nh;
    float w[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) w[u] = j0 + u < a.d ? nw[u] / (float)a.vm : 0.0f;
    if (it + gridDim.x < items) fetch(it + gridDim.x);
    int flag = 0;
    if (do_flow) {
      if (fabsf(h) * nrm <= rf) gst4(a.fl + it * MM, series_eval(T, s_g[0], h));
      else flag |= 1;
    }
    if (do_vl) {  // the knots on the series path (u_k, no P, V); or P, V on it with the knot chain; or neither
      const float c = h / (float)a.vm, x = fabsf(c) * nrm;
      if ((float)a.vm * x > rv) {
        flag |= 4;
        if (x <= rv) {
          gst4(a.vlm + it * 2 * MM, series_eval(T, s_g[1], c));
          gst4(a.vlm + it * 2 * MM + MM, series_eval(T, s_g[2], c));
        } else {
          flag |= 2;
        }
      } else {
        // u_k = A^k w: the thread's four columns of row i, summed over the row's 8 lanes (every lane gets each
        // sum); lane s of the 8 stores u_s, u_{s+8}, u_{s+16} of row i
        float pk[PW + 1];
#pragma unroll
        for (int k = 0; k <= PW; ++k)
          pk[k] = sum8(T[k].x * w[0] + T[k].y * w[1] + T[k].z * w[2] + T[k].w * w[3]);
        float o0 = pk[0], o1 = pk[8], o2 = pk[16];
#pragma unroll
        for (int q = 1; q < 8; ++q) {
          if (s8 == q) {
            o0 = pk[q];
            o1 = pk[8 + q];
            o2 = 16 + q <= PW ? pk[16 + q] : 0.0f;
          }
        }
        float* ub = a.ubuf + it * (PW + 1) * 32 + i;
        ub[s8 * 32] = o0;
        ub[(8 + s8) * 32] = o1;
        if (16 + s8 <= PW) ub[(16 + s8) * 32] = o2;
      }
    }
    if (threadIdx.x == 0) a.mflag[it] = flag;
  }
}

// per-sample step matrices (uniform reweighting modes) on the series path, a workgroup per sample: the shared flow
// (flow_mode cached / cached_basepoint) and the shared Van Loan pair; sflag[b] bit 0 (flow) / 1 (pair) flags a
// matrix outside the series radius, formed by k_wmat (mode 0) instead. An identity step (a zero or basepoint step)
// is never read and is not formed.
__global__ __launch_bounds__(NT) void k_wmat_series_smp(WArgs a) {
  __shared__ float s_g[3][PW + 1];
  if (threadIdx.x == 0) {
    series_gamma(a.chen, 0, s_g[0]);
    if (a.leaf == EWS_LEAF_VAN_LOAN) {
      series_gamma(a.vl_expm, 1, s_g[1]);
      series_gamma(a.vl_expm, 2, s_g[2]);
    }
  }
  __syncthreads();
  const int b = blockIdx.x;
  const float* th = a.clock + (size_t)b * a.L;
  const bool do_flow = a.flow_mode != EWS_FLOW_PER_INTERVAL;
  const bool do_vl = a.leaf == EWS_LEAF_VAN_LOAN && a.vl_mode != EWS_FLOW_PER_INTERVAL;
  float4 T[PW + 1];
  load_powers(a, T);
  const float nrm = a.apow[(size_t)(PW + 1) * MM];
  int flag = 0;
  if (do_flow) {
    bool ident;
    const float h = flow_step(a, th, 1, ident);
    if (!ident) {
      if (fabsf(h) * nrm <= series_radius(a.chen, 0)) gst4(a.fl + (size_t)b * MM, series_eval(T, s_g[0], h));
      else flag |= 1;
    }
  }
  if (do_vl) {
    bool fixed;
    const float c = vl_step(a, th, 1, fixed);
    if (!fixed) {
      if (fabsf(c) * nrm <= series_radius(a.vl_expm, 1)) {
        gst4(a.vlm + (size_t)b * 2 * MM, series_eval(T, s_g[1], c));
        gst4(a.vlm + (size_t)b * 2 * MM + MM, series_eval(T, s_g[2], c));
      } else {
        flag |= 2;
      }
    }
  }
  if (threadIdx.x == 0) a.sflag[b] = flag;
}

// sum over the workgroup of two values (every thread returns both; red: 2 NT / 64 floats); when cols, also each
// wavefront's column sums (lanes 0 .. 7, four columns each) into redw[wavefront][32] between the two barriers: they
// are read after the call returns and rewritten only after the next call's first barrier
__device__ __forceinline__ float2 block_sum2_cols(float u, float v, const float* dw, bool cols, float* red,
                                                  float* redw) {
  u = sum64(u);
  v = sum64(v);
  __syncthreads();
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  if (lane == 0) {
    red[wv] = u;
    red[NT / 64 + wv] = v;
  }
  if (cols && lane < 8)
    *reinterpret_cast<float4*>(redw + wv * 32 + lane * 4) = float4{dw[0], dw[1], dw[2], dw[3]};
  __syncthreads();
  float su = 0.0f, sv = 0.0f;
#pragma unroll
  for (int w = 0; w < NT / 64; ++w) {
    su += red[w];
    sv += red[NT / 64 + w];
  }
  return float2{su, sv};
}

// Adjoint of the series path: H_k partials of the workgroup (hpart) and the steps' cotangents (dhm) of every
// per-interval matrix not flagged; the flagged ones are k_wmat_bwd's (mode 2)
__global__ __launch_bounds__(NT) void k_wmat_bwd_series(WArgs a) {
  __shared__ float s_g[3][PW + 1];
  __shared__ float red[2 * NT / 64];
  __shared__ __align__(16) float redw[NT / 64][32];  // the series-path knots' dw, per wavefront
  if (threadIdx.x == 0) {
    series_gamma(a.chen, 0, s_g[0]);
    if (a.leaf == EWS_LEAF_VAN_LOAN) {
      series_gamma(a.vl_expm, 1, s_g[1]);
      series_gamma(a.vl_expm, 2, s_g[2]);
    }
  }
  __syncthreads();
  float4 T[PW + 1], H[PW + 1];
  load_powers(a, T);
#pragma unroll
  for (int k = 0; k <= PW; ++k) H[k] = float4{0.0f, 0.0f, 0.0f, 0.0f};
  const bool do_flow = a.flow_mode == EWS_FLOW_PER_INTERVAL;
  const bool do_vl = a.leaf == EWS_LEAF_VAN_LOAN && a.vl_mode == EWS_FLOW_PER_INTERVAL;
  const long items = (long)a.B * a.n;
  const int i = trow<32>(), j0 = tcol<32>();
  // the next item's clock step and flags, loaded during the item before
  float nh = 0.0f;
  int nflag = 0;
  auto fetch = [&](long it) {
    const int b = (int)(it / a.n), t = (int)(it - (long)b * a.n);
    nh = a.clock[(size_t)b * a.L + t + 1] - a.clock[(size_t)b * a.L + t];
    nflag = a.mflag[it];
  };
  if ((long)blockIdx.x < items) fetch(blockIdx.x);
  for (long it = blockIdx.x; it < items; it += gridDim.x) {
    const int b = (int)(it / a.n), t = (int)(it - (long)b * a.n);
    const float h = nh;
    const int flag = nflag;
    // sv: the Van Loan pair on the series path (its knots by the chain); sk: the knots themselves on it (their
    // clock-step cotangent is the leaf adjoint's)
    const bool sf = do_flow && !(flag & 1), sv = do_vl && (flag & 4) && !(flag & 2), sk = do_vl && !(flag & 4);
    // every load of the item issued before its first use
    float4 G = float4{0.0f, 0.0f, 0.0f, 0.0f}, GP = G, GV = G;
    float ek[PW + 1], xv[4];
    if (sf) G = gld4(a.dfl + it * MM);
    if (sv) {
      GP = gld4(a.dvlm + it * 2 * MM);
      GV = gld4(a.dvlm + it * 2 * MM + MM);
    }
    if (sk) {
      const float* e = a.ebuf + (size_t)it * (PW + 1) * 32 + i;
#pragma unroll
      for (int k = 0; k <= PW; ++k) ek[k] = e[k * 32];
      const float* x = a.path + ((size_t)b * a.L + t) * a.d;
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int j = min(j0 + u, a.d - 1);  // in bounds; the padded columns are zeroed below
        xv[u] = x[a.d + j] - x[j];
      }
    }
    if (it + gridDim.x < items) fetch(it + gridDim.x);
    float df = 0.0f, dv = 0.0f;
    if (sf) {  // H_k += gamma_k h^k G; dh = <G, sum_k k gamma_k h^(k-1) A^k>
      float ck = 1.0f, dk = 0.0f;  // h^k, k h^(k-1)
#pragma unroll
      for (int k = 0; k <= PW; ++k) {
        const float w = s_g[0][k] * ck, wd = s_g[0][k] * dk;
        H[k].x = fmaf(w, G.x, H[k].x);
        H[k].y = fmaf(w, G.y, H[k].y);
        H[k].z = fmaf(w, G.z, H[k].z);
        H[k].w = fmaf(w, G.w, H[k].w);
        // the weight first: with large cotangents, <G, A^k> alone can overflow where the weight is zero or tiny
        df += (wd * G.x) * T[k].x + (wd * G.y) * T[k].y + (wd * G.z) * T[k].z + (wd * G.w) * T[k].w;
        dk = fmaf(dk, h, ck);
        ck *= h;
      }
    }
    if (sv) {
      const float c = h / (float)a.vm;
      float ck = 1.0f, dk = 0.0f;
#pragma unroll
      for (int k = 0; k <= PW; ++k) {
        const float wp = s_g[1][k], wv = s_g[2][k];
        const float4 G = float4{wp * GP.x + wv * GV.x, wp * GP.y + wv * GV.y, wp * GP.z + wv * GV.z,
                                wp * GP.w + wv * GV.w};
        H[k].x = fmaf(ck, G.x, H[k].x);
        H[k].y = fmaf(ck, G.y, H[k].y);
        H[k].z = fmaf(ck, G.z, H[k].z);
        H[k].w = fmaf(ck, G.w, H[k].w);
        dv += (dk * G.x) * T[k].x + (dk * G.y) * T[k].y + (dk * G.z) * T[k].z + (dk * G.w) * T[k].w;
        dk = fmaf(dk, c, ck);
        ck *= c;
      }
    }
    float dw[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if (sk) {
      // knots sum_k phi[m][k] c^k A^k w with e_k their cotangents: H_k += c^k e_k w^T, dw = sum_k c^k (A^k)^T e_k
      // (the thread's row-i part of its four columns), dc = sum_k k c^(k-1) <e_k, A^k w> (into dv); w = v / M
      const float c = h / (float)a.vm;
      float w[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) w[u] = j0 + u < a.d ? xv[u] / (float)a.vm : 0.0f;
      float ck = 1.0f, dk = 0.0f;  // c^k, k c^(k-1)
#pragma unroll
      for (int k = 0; k <= PW; ++k) {
        const float cek = ck * ek[k];
        H[k].x = fmaf(cek, w[0], H[k].x);
        H[k].y = fmaf(cek, w[1], H[k].y);
        H[k].z = fmaf(cek, w[2], H[k].z);
        H[k].w = fmaf(cek, w[3], H[k].w);
        dw[0] = fmaf(cek, T[k].x, dw[0]);
        dw[1] = fmaf(cek, T[k].y, dw[1]);
        dw[2] = fmaf(cek, T[k].z, dw[2]);
        dw[3] = fmaf(cek, T[k].w, dw[3]);
        dv = fmaf(dk * ek[k], T[k].x * w[0] + T[k].y * w[1] + T[k].z * w[2] + T[k].w * w[3], dv);
        dk = fmaf(dk, c, ck);
        ck *= c;
      }
      // over the wavefront's 8 rows (lanes 8 apart hold the same columns): lanes 0 .. 7 keep the sums
#pragma unroll
      for (int u = 0; u < 4; ++u) dw[u] = colsum8(dw[u]);
    }
    if (sf || sv || sk) {  // uniform over the workgroup
      const float2 s2 = block_sum2_cols(df, dv, dw, sk, red, &redw[0][0]);
      if (threadIdx.x == 0) {
        if (sf) a.dhm[2 * it] = s2.x;
        if (sv || sk) a.dhm[2 * it + 1] = s2.y / (float)a.vm;  // c = h / M
      }
      if (sk && threadIdx.x < a.d) {  // the wavefronts' column sums, in order: dv = dw / M
        float sw = 0.0f;
#pragma unroll
        for (int wv = 0; wv < NT / 64; ++wv) sw += redw[wv][threadIdx.x];
        a.dv[(size_t)it * DP + threadIdx.x] = sw / (float)a.vm;
      }
    }
  }
#pragma unroll
  for (int k = 0; k <= PW; ++k) gst4(a.hpart + ((size_t)blockIdx.x * (PW + 1) + k) * MM, H[k]);
}

// Adjoint of the per-sample series path, a workgroup per sample: the shared flow's cotangent (its chunks' partials)
// and the shared pair's (its leaf slices' partials), summed in order as k_wmat_bwd does, into the sample's H_k slot
// (hpart slot hslot0 + b) and the shared steps' cotangents dsh[b]; flagged matrices are k_wmat_bwd's (mode 0)
__global__ __launch_bounds__(NT) void k_wmat_bwd_series_smp(WArgs a, int hslot0) {
  __shared__ float s_g[3][PW + 1];
  __shared__ float red[2 * NT / 64];
  if (threadIdx.x == 0) {
    series_gamma(a.chen, 0, s_g[0]);
    if (a.leaf == EWS_LEAF_VAN_LOAN) {
      series_gamma(a.vl_expm, 1, s_g[1]);
      series_gamma(a.vl_expm, 2, s_g[2]);
    }
  }
  __syncthreads();
  const int b = blockIdx.x;
  const float* th = a.clock + (size_t)b * a.L;
  const int flag = a.sflag[b];
  const bool do_flow = a.flow_mode != EWS_FLOW_PER_INTERVAL && !(flag & 1);
  const bool do_vl = a.leaf == EWS_LEAF_VAN_LOAN && a.vl_mode != EWS_FLOW_PER_INTERVAL && !(flag & 2);
  float4 T[PW + 1], H[PW + 1];
  load_powers(a, T);
#pragma unroll
  for (int k = 0; k <= PW; ++k) H[k] = float4{0.0f, 0.0f, 0.0f, 0.0f};
  float df = 0.0f, dv = 0.0f;
  bool sf = false, sv = false;
  if (do_flow) {
    bool ident;
    const float h = flow_step(a, th, 1, ident);
    sf = true;
    float4 G = float4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll 8
    for (int c = 0; c < a.C; ++c) G = f4add(G, gld4(a.cpart + ((size_t)b * a.CP + c) * 3 * MM));
    float ck = 1.0f, dk = 0.0f;  // h^k, k h^(k-1)
#pragma unroll
    for (int k = 0; k <= PW; ++k) {
      const float w = s_g[0][k] * ck, wd = s_g[0][k] * dk;
      H[k].x = fmaf(w, G.x, H[k].x);
      H[k].y = fmaf(w, G.y, H[k].y);
      H[k].z = fmaf(w, G.z, H[k].z);
      H[k].w = fmaf(w, G.w, H[k].w);
      df += (wd * G.x) * T[k].x + (wd * G.y) * T[k].y + (wd * G.z) * T[k].z + (wd * G.w) * T[k].w;
      dk = fmaf(dk, h, ck);
      ck *= h;
    }
  }
  if (do_vl) {
    bool fixed;
    const float c = vl_step(a, th, 1, fixed);
    if (!fixed) {
      sv = true;
      float4 GP = float4{0.0f, 0.0f, 0.0f, 0.0f}, GV = GP;
#pragma unroll 8
      for (int s2 = 0; s2 < a.NSL; ++s2) {
        const float* cp = a.cpart + ((size_t)b * a.CP + s2) * 3 * MM;
        GP = f4add(GP, gld4(cp + MM));
        GV = f4add(GV, gld4(cp + 2 * MM));
      }
      float ck = 1.0f, dk = 0.0f;
#pragma unroll
      for (int k = 0; k <= PW; ++k) {
        const float wp = s_g[1][k], wv = s_g[2][k];
        const float4 G = float4{wp * GP.x + wv * GV.x, wp * GP.y + wv * GV.y, wp * GP.z + wv * GV.z,
                                wp * GP.w + wv * GV.w};
        H[k].x = fmaf(ck, G.x, H[k].x);
        H[k].y = fmaf(ck, G.y, H[k].y);
        H[k].z = fmaf(ck, G.z, H[k].z);
        H[k].w = fmaf(ck, G.w, H[k].w);
        dv += (dk * G.x) * T[k].x + (dk * G.y) * T[k].y + (dk * G.z) * T[k].z + (dk * G.w) * T[k].w;
        dk = fmaf(dk, c, ck);
        ck *= c;
      }
    }
  }
  const float dw0[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  const float2 s2 = block_sum2_cols(df, dv, dw0, false, red, nullptr);
  if (threadIdx.x == 0) {
    if (sf) a.dsh[2 * b] = s2.x;
    if (sv) a.dsh[2 * b + 1] = s2.y / (float)a.vm;  // c = dt / M
  }
#pragma unroll
  for (int k = 0; k <= PW; ++k) gst4(a.hpart + ((size_t)(hslot0 + b) * (PW + 1) + k) * MM, H[k]);
}

// H_k summed over the workgroups' partials (float64, a fixed order): a workgroup per (k, 64 entries); its four
// wavefronts take the partials g = 4 q + w (two running sums each, even and odd q), then wavefront 0 adds the
// eight sums in order
__global__ __launch_bounds__(NT) void k_whsum(WArgs a, int nparts) {
  __shared__ double red[NT / 64][2][64];
  const int k = blockIdx.x, lane = threadIdx.x & 63, w = threadIdx.x >> 6, e = blockIdx.y * 64 + lane;
  const float* src = a.hpart + (size_t)k * MM + e;
  const size_t stride = (size_t)(PW + 1) * MM;
  double s0 = 0.0, s1 = 0.0;
  int g = w;
  for (; g + 4 < nparts; g += 8) {
    s0 += (double)src[(size_t)g * stride];
    s1 += (double)src[(size_t)(g + 4) * stride];
  }
  if (g < nparts) s0 += (double)src[(size_t)g * stride];
  red[w][0][lane] = s0;
  red[w][1][lane] = s1;
  __syncthreads();
  if (w == 0) {
    double s = 0.0;
#pragma unroll
    for (int q = 0; q < NT / 64; ++q) s += red[q][0][lane] + red[q][1][lane];
    a.hsum[(size_t)k * MM + e] = s;
  }
}

// dA of the series path (float64): R_{PW-1} = H_PW, R_i = H_{i+1} + R_{i+1} A^T, U_i = R_i + A^T U_{i+1},
// dA = U_0; into apart slot `slot`
__global__ __launch_bounds__(NT) void k_wseries_dA(WArgs a, long slot) {
  __shared__ __align__(16) double sd[3 * S32];
  double* A = sd;
  double* R = sd + S32;
  double* U = sd + 2 * S32;
  load_A(a.d, a.A, A);
  const v4d z = v4d{0.0, 0.0, 0.0, 0.0};
  st_tile_d(R, z);
  st_tile_d(U, z);
  __syncthreads();
  const int tn = tile_n0() + tile_i();  // the lane's tile entries: rows tile_row_d(r) of column tn
  v4d u = z;
  for (int ii = PW - 1; ii >= 0; --ii) {
    v4d r = mm_tile_d<false, true>(R, A, z);  // R A^T
    u = mm_tile_d<true, false>(A, U, z);      // A^T U
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      r[c] += a.hsum[(size_t)(ii + 1) * MM + tile_row_d(c) * DP + tn];
      u[c] += r[c];
    }
    __syncthreads();
    st_tile_d(U, u);
    st_tile_d(R, r);
    __syncthreads();
  }
#pragma unroll
  for (int c = 0; c < 4; ++c) a.apart[slot * MM + tile_row_d(c) * DP + tn] = (float)u[c];
}

// The thread's four entries of the flow of interval t of sample b (registers), and their store into F and, transposed,
// Ft (LDS): the scans load a step's operands into registers during the step before it.
__device__ __forceinline__ float4 flow_regs(const WArgs& a, int b, int t) {
  bool ident;
  flow_step(a, a.clock + (size_t)b * a.L, t, ident);
  if (ident) {
    const int i = trow<32>(), j0 = tcol<32>();
    return float4{i == j0 ? 1.0f : 0.0f, i == j0 + 1 ? 1.0f : 0.0f, i == j0 + 2 ? 1.0f : 0.0f,
                  i == j0 + 3 ? 1.0f : 0.0f};
  }
  const size_t item = a.flow_mode == EWS_FLOW_PER_INTERVAL ? (size_t)b * a.n + t : (size_t)b;
  return gld4(a.fl + item * MM);
}
__device__ __forceinline__ void commit_mat(float4 v, float* F, float* Ft) {
  sld4(F, v);
  const int i = trow<32>(), j0 = tcol<32>();
  Ft[(j0 + 0) * P32 + i] = v.x;
  Ft[(j0 + 1) * P32 + i] = v.y;
  Ft[(j0 + 2) * P32 + i] = v.z;
  Ft[(j0 + 3) * P32 + i] = v.w;
}

// ------------------------------------------------------------------------------------------------ local terms
// LDS of the leaf kernels (floats): A, P, V (32 x 36 each), vectors, the knot / letter table and its cotangents.
// The four tables hold `rows` rows of 32 (the knots M or the letters q + 1), in dynamic LDS sized to them:
// knots Delta_m (or letters b_p); Y_m (or u_p); R_m, Pre_m (or w_p, A b_{p-1}); cotangents.
constexpr int LF_A = 0, LF_P = S32, LF_V = 2 * S32, LF_S2 = 3 * S32, LF_VEC = 4 * S32;  // vectors: 8 x 32
constexpr int LF_TAB = LF_VEC + 8 * 32;
__host__ __device__ constexpr int lf_floats(int rows, int ntab) { return LF_TAB + ntab * rows * 32 + 64; }
// with a per-interval Van Loan leaf: phi (M rows of PW + 1) and u_k = A^k w (PW + 1 rows of 32)
constexpr int LX_PHI = 64 * (PW + 1), LX_U = (PW + 1) * 32;
constexpr int LF_EXTRA = LX_PHI + LX_U;

// knots Delta_1 .. Delta_M into D (rows 0 .. M-1) on the series path: Delta_{r+1} = sum_k phi[r][k] c^k u_k from
// u_k = A^k w (rows of U, formed per interval by k_wmat_series)
__device__ void series_knots(int M, const float* phi, const float* U, float* D, float c) {
  const int tid = threadIdx.x;
  for (int e = tid; e < M * 32; e += NT) {
    const int r = e >> 5, row = e & 31;
    float x = 0.0f, ck = 1.0f;
#pragma unroll 4
    for (int k = 0; k <= PW; ++k) {
      x = fmaf(phi[r * (PW + 1) + k] * ck, U[k * 32 + row], x);
      ck *= c;
    }
    D[e] = x;
  }
  __syncthreads();
}

// the knots' partial sums, 8 lanes per channel (a segment of ceil(M / 8) knots each, scanned across the 8 lanes):
// Y_m = Pre_m + Delta_m / 2 (Pre_m the knots before m), Z_m = R_m + Delta_m / 2 (R_m the knots after m, when Z is
// given) and s1 = sum_m Delta_m (into s1 when given); D, Y, Z hold rows m of 32
__device__ void knot_sums(int M, const float* D, float* Y, float* Z, float* s1) {
  const int tid = threadIdx.x, col = tid >> 3, seg = tid & 7;
  const int S = (M + 7) >> 3, m0 = min(M, seg * S), m1 = min(M, m0 + S);
  float own = 0.0f;
  for (int m = m0; m < m1; ++m) own += D[m * 32 + col];
  float inc = own;
#pragma unroll
  for (int o = 1; o < 8; o <<= 1) {
    const float v = __shfl_up(inc, o, 8);
    if (seg >= o) inc += v;
  }
  const float total = __shfl(inc, 7, 8);
  float pre = inc - own;
  for (int m = m0; m < m1; ++m) {
    const float dm = D[m * 32 + col];
    Y[m * 32 + col] = fmaf(0.5f, dm, pre);
    pre += dm;
  }
  if (Z) {
    float suf = total - inc;
    for (int m = m1 - 1; m >= m0; --m) {
      const float dm = D[m * 32 + col];
      Z[m * 32 + col] = fmaf(0.5f, dm, suf);
      suf += dm;
    }
  }
  if (s1 && seg == 0) s1[col] = total;
}

__device__ __forceinline__ float inv_f(int n) { return 1.0f / (float)n; }
__device__ __forceinline__ float c2coef(int p, int r) { return 1.0f / ((float)(p + r + 2) * (float)(r + 1)); }

// knots of the interval: Delta_M = V w, Delta_{m-1} = P Delta_m (rows 0 .. M-1 of D hold Delta_1 .. Delta_M),
// w = v / M in wv
__device__ void vl_knots(const WArgs& a, const float* P, const float* V, const float* wv, float* D) {
  const int M = a.vm, i = (int)threadIdx.x >> 3;
  float y = mv<false>(V, wv);
  if (threadIdx.x < 256 && row_lead()) D[(M - 1) * 32 + i] = y;
  __syncthreads();
  for (int m = M - 1; m >= 1; --m) {
    y = mv<false>(P, D + m * 32);
    if (row_lead()) D[(m - 1) * 32 + i] = y;
    __syncthreads();
  }
}

// interval's local terms (s1 into s1v, s2 into the thread's registers) from its inputs staged in LDS: the increment
// (divided by M for the Van Loan leaf) in vec; P, V (the Van Loan leaf off the series path) or u_k (on it, ser)
template <int N>
__device__ void leaf_fwd(const WArgs& a, float* sm, float h, float* s1v, float* s2r, bool ser) {
  float* vec = sm + LF_VEC;
  float* T1 = sm + LF_TAB;
  float* T2 = T1 + (a.leaf == EWS_LEAF_VAN_LOAN ? a.vm : a.q + 1) * 32;
  const int tid = threadIdx.x, i = tid >> 3, j0 = (tid & 7) * 4;
  if (a.leaf == EWS_LEAF_VAN_LOAN) {
    if (ser) {
      float* phi = sm + lf_floats(a.vm, 2);
      series_knots(a.vm, phi, phi + LX_PHI, T1, h / (float)a.vm);
    } else {
      vl_knots(a, sm + LF_P, sm + LF_V, vec, T1);
    }
    const int M = a.vm;
    knot_sums(M, T1, T2, nullptr, s1v);  // s1 and Y_m = Pre_m + Delta_m / 2
    __syncthreads();
    if constexpr (N >= 2) {  // s2 = sum_m Y_m Delta_m^T
#pragma unroll
      for (int c = 0; c < 4; ++c) s2r[c] = 0.0f;
      for (int m = 0; m < M; ++m) {
        const float y = T2[m * 32 + i];
        const float4 dl = *reinterpret_cast<const float4*>(T1 + m * 32 + j0);
        s2r[0] = fmaf(y, dl.x, s2r[0]);
        s2r[1] = fmaf(y, dl.y, s2r[1]);
        s2r[2] = fmaf(y, dl.z, s2r[2]);
        s2r[3] = fmaf(y, dl.w, s2r[3]);
      }
    }
  } else {
    // letters b_p (rows of T1), u_p = sum_{r <= q-p} C2[p][r] b_r (rows of T2)
    const int q = a.q;
    float* A = sm + LF_A;
    if (tid < 32) T1[tid] = vec[tid];
    __syncthreads();
    for (int p = 1; p <= q; ++p) {
      const float y = mv<false>(A, T1 + (p - 1) * 32);
      if (row_lead()) T1[p * 32 + i] = (-h / (float)p) * y;
      __syncthreads();
    }
    if (tid < 32) {
      float s = 0.0f;
      for (int p = 0; p <= q; ++p) s = fmaf(inv_f(p + 1), T1[p * 32 + tid], s);
      s1v[tid] = s;
    }
    if constexpr (N >= 2) {
      for (int e = tid; e < (q + 1) * 32; e += NT) {
        const int p = e >> 5, k = e & 31;
        float s = 0.0f;
        for (int r = 0; r <= q - p; ++r) s = fmaf(c2coef(p, r), T1[r * 32 + k], s);
        T2[p * 32 + k] = s;
      }
      __syncthreads();
#pragma unroll
      for (int c = 0; c < 4; ++c) s2r[c] = 0.0f;
      for (int p = 0; p <= q; ++p) {  // s2 = sum_p b_p u_p^T
        const float y = T1[p * 32 + i];
        const float4 u = *reinterpret_cast<const float4*>(T2 + p * 32 + j0);
        s2r[0] = fmaf(y, u.x, s2r[0]);
        s2r[1] = fmaf(y, u.y, s2r[1]);
        s2r[2] = fmaf(y, u.z, s2r[2]);
        s2r[3] = fmaf(y, u.w, s2r[3]);
      }
    }
  }
  __syncthreads();
}

// SER: the per-interval Van Loan leaf, whose knots may take the series path (a separate instantiation keeps the
// other leaves' register count low). Each interval's inputs are loaded into registers during the interval before.
template <int N, bool SER>
__global__ __launch_bounds__(NT) void k_wleaf(WArgs a) {
  extern __shared__ __align__(16) float sm[];  // lf_floats(rows, 2) (+ LF_EXTRA, per-interval Van Loan)
  float* vec = sm + LF_VEC;
  float* s1v = sm + LF_VEC + 32;
  float* P = sm + LF_P;
  float* V = sm + LF_V;
  float* Ub = sm + lf_floats(a.vm, 2) + LX_PHI;  // u_k (SER)
  const int tid = threadIdx.x;
  load_A(a.d, a.A, sm + LF_A);
  if (SER) {  // the knots' coefficients of the series path
    float* phi = sm + lf_floats(a.vm, 2);
    for (int e = tid; e < a.vm * (PW + 1); e += NT) phi[e] = a.apow[PHI_OFF + e];
  }
  const bool vl = a.leaf == EWS_LEAF_VAN_LOAN;
  const bool vl_int = vl && a.vl_mode == EWS_FLOW_PER_INTERVAL;
  const long items = (long)a.B * a.n;
  float nv = 0.0f, nh = 0.0f, nU[3] = {0.0f, 0.0f, 0.0f};  // (PW + 1) * 32 <= 3 NT
  float4 nP = float4{0.0f, 0.0f, 0.0f, 0.0f}, nV = nP;
  bool nser = false, nfixed = false;
  auto fetch = [&](long it) {
    const int b = (int)(it / a.n), t = (int)(it - (long)b * a.n);
    const float* x = a.path + ((size_t)b * a.L + t) * a.d;
    const float* th = a.clock + (size_t)b * a.L;
    if (tid < 32) nv = tid < a.d ? x[a.d + tid] - x[tid] : 0.0f;
    nh = th[t + 1] - th[t];
    if (vl) {
      nser = SER && !(a.mflag[it] & 4);
      if (nser) {
#pragma unroll
        for (int k = 0; k < 3; ++k) {
          const int e = tid + k * NT;
          nU[k] = e < (PW + 1) * 32 ? a.ubuf[it * (PW + 1) * 32 + e] : 0.0f;
        }
      } else {
        bool fixed;
        vl_step(a, th, t, fixed);
        nfixed = fixed && !vl_int;
        if (!nfixed) {
          const size_t item = vl_int ? (size_t)it : (size_t)b;
          nP = gld4(a.vlm + item * 2 * MM);
          nV = gld4(a.vlm + item * 2 * MM + MM);
        }
      }
    }
  };
  if ((long)blockIdx.x < items) fetch(blockIdx.x);
  for (long it = blockIdx.x; it < items; it += gridDim.x) {
    const bool ser = nser;
    const float h = nh;
    if (tid < 32) vec[tid] = vl ? nv / (float)a.vm : nv;
    if (vl) {
      if (ser) {
#pragma unroll
        for (int k = 0; k < 3; ++k) {
          const int e = tid + k * NT;
          if (e < (PW + 1) * 32) Ub[e] = nU[k];
        }
      } else if (nfixed) {
        set_ident32(P, 1.0f);
        set_ident32(V, 1.0f);
      } else {
        sld4(P, nP);
        sld4(V, nV);
      }
    }
    __syncthreads();
    if (it + gridDim.x < items) fetch(it + gridDim.x);
    float s2r[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    leaf_fwd<N>(a, sm, h, s1v, s2r, ser);
    float* row = a.loc + it * RW;
    if (tid < 32) row[tid] = s1v[tid];
    if constexpr (N >= 2) gst4(row + DP, acc4(s2r));
    __syncthreads();
  }
}

// ------------------------------------------------------------------------------------------------ Chen scan
constexpr int SC_F = 0, SC_FT = S32, SC_S2 = 2 * S32, SC_T = 3 * S32, SC_PH = 4 * S32, SC_PN = 5 * S32;
constexpr int SC_VEC = 6 * S32;  // S1, y1, s1 (32 each)
constexpr int SC_FLOATS = SC_VEC + 3 * 32;

// one Chen step of the state (S1, S2) in LDS by (F, Ft, s1 in LDS; s2 the lane's tile entries); with PHI the flow
// product Ph <- F Ph as well (Pn scratch; the pointers swap). The three products run on MFMA, over the first ku
// k-steps where a factor is a state (zero past d).
template <int N, bool PHI>
__device__ __forceinline__ void chen_step(float* sm, const v4f s2, float*& Ph, float*& Pn, int ku) {
  float* F = sm + SC_F;
  float* Ft = sm + SC_FT;
  float* S2 = sm + SC_S2;
  float* T = sm + SC_T;
  float* S1 = sm + SC_VEC;
  float* y1 = S1 + 32;
  float* s1 = S1 + 64;
  const int i = (int)threadIdx.x >> 3;
  const float y = mv<false>(F, S1);
  if constexpr (N >= 2) st_tile(T, mm_tile<false, false>(F, S2, zero4(), ku));
  if constexpr (PHI) st_tile(Pn, mm_tile<false, false>(F, Ph, zero4()));  // (all of K: Ph's padding is I)
  if (row_lead()) y1[i] = y;
  __syncthreads();
  if constexpr (N >= 2) {  // S2 <- F S2 F^T + y1 s1^T + s2 (S2 is not read in this phase)
    v4f acc = mm_tile<false, false>(T, Ft, s2, ku);
    const int m = tile_m0() + 4 * tile_g(), n = tile_n0() + tile_i();
    const float sn = s1[n];
#pragma unroll
    for (int r = 0; r < 4; ++r) acc[r] = fmaf(y1[m + r], sn, acc[r]);
    st_tile(S2, acc);
  }
  if (row_lead()) S1[i] = y + s1[i];
  if constexpr (PHI) {
    float* tmp = Ph;
    Ph = Pn;
    Pn = tmp;
  }
  __syncthreads();
}

__device__ __forceinline__ void load_state(const float* g, float* S1, float* S2) {
  if (threadIdx.x < 32) S1[threadIdx.x] = g[threadIdx.x];
  sld4(S2, gld4(g + DP));
}
__device__ __forceinline__ void store_state(float* g, const float* S1, const float* S2) {
  if (threadIdx.x < 32) g[threadIdx.x] = S1[threadIdx.x];
  gst4(g + DP, lds4(S2));
}

// the packed output row (level 0, S1[:d], S2[:d, :d]) of the state in LDS
template <int N>
__device__ __forceinline__ void store_packed(const WArgs& a, float* o, const float* S1, const float* S2) {
  const int d = a.d;
  if (a.lvl0 && threadIdx.x == 0) o[0] = 1.0f;
  o += a.lvl0;
  if ((int)threadIdx.x < d) o[threadIdx.x] = S1[threadIdx.x];
  if constexpr (N >= 2) {
    for (int e = threadIdx.x; e < d * d; e += NT) {
      const int r = e / d, c = e - r * d;
      o[d + e] = S2[r * P32 + c];
    }
  }
}

constexpr int SCAN_SUMMARY = 0, SCAN_ROWS = 1;

template <int N, int MODE>
__global__ __launch_bounds__(NT) void k_wscan(WArgs a) {
  const int ku = (a.d + 3) >> 2;  // MFMA k-steps that reach a nonzero entry (d <= 4 ku)
  __shared__ __align__(16) float sm[SC_FLOATS];
  const int c = blockIdx.x, b = blockIdx.y;
  const int t0 = c * a.T, t1 = min(a.n, t0 + a.T);
  float* S1 = sm + SC_VEC;
  float* S2 = sm + SC_S2;
  float* s1 = S1 + 64;
  float* Ph = sm + SC_PH;
  float* Pn = sm + SC_PN;
  if (MODE == SCAN_SUMMARY) {
    if (threadIdx.x < 32) S1[threadIdx.x] = 0.0f;
    sld4(S2, float4{0.0f, 0.0f, 0.0f, 0.0f});
    set_ident32(Ph, 1.0f);
  } else {
    load_state(a.car + ((size_t)b * (a.C + 1) + c) * RW, S1, S2);
  }
  // the step's flow, s1 and s2 in registers, loaded during the step before
  float4 nF = flow_regs(a, b, t0);
  v4f ns2 = zero4();
  float ns1 = 0.0f;
  auto fetch = [&](int t) {
    const float* lrow = a.loc + ((size_t)b * a.n + t) * RW;
    if (threadIdx.x < 32) ns1 = lrow[threadIdx.x];
    if (N >= 2) ns2 = gld_tile(lrow + DP);
  };
  fetch(t0);
  // mean / max readout: the chunk's sum, or its maximum and the first row attaining it, of the thread's padded
  // entries (level 1: threads below 32; level 2: row i, columns j0 .. j0 + 3)
  const bool mean = a.readout == EWS_READOUT_MEAN, mx = a.readout == EWS_READOUT_MAX;
  float p1 = mean ? 0.0f : -INFINITY, p2[4] = {p1, p1, p1, p1};
  int i1 = -1, i2[4] = {-1, -1, -1, -1};
  for (int t = t0; t < t1; ++t) {
    commit_mat(nF, sm + SC_F, sm + SC_FT);
    if (threadIdx.x < 32) s1[threadIdx.x] = ns1;
    const v4f s2 = ns2;
    __syncthreads();
    if (t + 1 < t1) {
      nF = flow_regs(a, b, t + 1);
      fetch(t + 1);
    }
    chen_step<N, MODE == SCAN_SUMMARY>(sm, s2, Ph, Pn, ku);
    if constexpr (MODE == SCAN_ROWS) {
      const size_t r = (size_t)b * a.n + t;
      if (a.rows) store_state(a.rows + r * RW, S1, S2);
      if (a.readout == EWS_READOUT_PREFIX) store_packed<N>(a, a.out + r * a.W, S1, S2);
      if (mean || mx) {
        const float v1 = threadIdx.x < 32 ? S1[threadIdx.x] : 0.0f;
        const float4 v2 = N >= 2 ? lds4(S2) : float4{0.0f, 0.0f, 0.0f, 0.0f};
        const float v[4] = {v2.x, v2.y, v2.z, v2.w};
        if (mean) {
          p1 += v1;
#pragma unroll
          for (int u = 0; u < 4; ++u) p2[u] += v[u];
        } else {
          if (i1 < 0 || v1 > p1) {
            p1 = v1;
            i1 = t;
          }
#pragma unroll
          for (int u = 0; u < 4; ++u) {
            if (i2[u] < 0 || v[u] > p2[u]) {
              p2[u] = v[u];
              i2[u] = t;
            }
          }
        }
      }
    }
  }
  if constexpr (MODE == SCAN_ROWS) {
    if (mean || mx) {
      const size_t slot = ((size_t)b * a.C + c) * RW;
      if (threadIdx.x < 32) a.rpart[slot + threadIdx.x] = p1;
      if constexpr (N >= 2) gst4(a.rpart + slot + DP, float4{p2[0], p2[1], p2[2], p2[3]});
      if (mx) {
        if (threadIdx.x < 32) a.ridx[slot + threadIdx.x] = i1;
        if constexpr (N >= 2) {
          int* q = a.ridx + slot + DP + trow<32>() * DP + tcol<32>();
#pragma unroll
          for (int u = 0; u < 4; ++u) q[u] = i2[u];
        }
      }
    }
  }
  if (MODE == SCAN_SUMMARY) {
    store_state(a.summ + ((size_t)b * a.C + c) * RW, S1, S2);
    gst4(a.sfl + ((size_t)b * a.C + c) * MM, lds4(Ph));
  }
}

// carries: car[b][0] = 0, car[b][c + 1] = the chunk-c Chen map of car[b][c] (flow product and summary)
template <int N>
__global__ __launch_bounds__(NT) void k_wcarry(WArgs a) {
  const int ku = (a.d + 3) >> 2;  // MFMA k-steps that reach a nonzero entry (d <= 4 ku)
  __shared__ __align__(16) float sm[SC_FLOATS];
  const int b = blockIdx.x;
  float* S1 = sm + SC_VEC;
  float* S2 = sm + SC_S2;
  float* s1 = S1 + 64;
  float* F = sm + SC_F;
  float* Ft = sm + SC_FT;
  if (threadIdx.x < 32) S1[threadIdx.x] = 0.0f;
  sld4(S2, float4{0.0f, 0.0f, 0.0f, 0.0f});
  __syncthreads();
  float* car = a.car + (size_t)b * (a.C + 1) * RW;
  store_state(car, S1, S2);
  float* dummy0 = nullptr;
  float* dummy1 = nullptr;
  for (int c = 0; c < a.C; ++c) {
    commit_mat(gld4(a.sfl + ((size_t)b * a.C + c) * MM), F, Ft);
    const float* sr = a.summ + ((size_t)b * a.C + c) * RW;
    if (threadIdx.x < 32) s1[threadIdx.x] = sr[threadIdx.x];
    const v4f s2 = N >= 2 ? gld_tile(sr + DP) : zero4();
    __syncthreads();
    chen_step<N, false>(sm, s2, dummy0, dummy1, ku);
    store_state(car + (size_t)(c + 1) * RW, S1, S2);
  }
}

// terminal / mean / max readouts: a workgroup per (sample, 32 packed columns); the mean and max run over the rows in
// 8 interleaved groups combined in a fixed order (the max keeps the first row attaining it)
constexpr int RO_COLS = 32, RO_GROUPS = NT / RO_COLS;
__global__ __launch_bounds__(NT) void k_wreadout(WArgs a) {
  __shared__ float s_v[RO_GROUPS][RO_COLS];
  __shared__ int s_i[RO_GROUPS][RO_COLS];
  const int b = blockIdx.y, cl = threadIdx.x % RO_COLS, grp = threadIdx.x / RO_COLS;
  const int col = blockIdx.x * RO_COLS + cl;
  const bool ok = col < a.W;
  float* o = a.out + (size_t)b * a.W;
  const int e = col - a.lvl0, d = a.d;
  const int pe = !ok || e < 0 ? 0 : (e < d ? e : DP + ((e - d) / d) * DP + (e - d) % d);  // padded index
  if (a.readout == EWS_READOUT_TERMINAL) {
    if (ok && grp == 0) o[col] = e < 0 ? 1.0f : a.car[((size_t)b * (a.C + 1) + a.C) * RW + pe];
    return;
  }
  // the chunks' partials (k_wscan rows pass) in 8 interleaved groups of chunks
  const float* r = a.rpart + (size_t)b * a.C * RW + pe;
  const int* ri = a.ridx ? a.ridx + (size_t)b * a.C * RW + pe : nullptr;
  float acc = a.readout == EWS_READOUT_MEAN ? 0.0f : -INFINITY;
  int arg = -1;
  for (int c = grp; c < a.C; c += RO_GROUPS) {
    const float v = ok ? r[(size_t)c * RW] : 0.0f;
    if (a.readout == EWS_READOUT_MEAN) {
      acc += v;
    } else if (arg < 0 || v > acc) {  // chunks in order: the first row attaining the maximum is kept
      acc = v;
      arg = ok ? ri[(size_t)c * RW] : 0;
    }
  }
  s_v[grp][cl] = acc;
  s_i[grp][cl] = arg;
  __syncthreads();
  if (grp != 0 || !ok) return;
  if (e < 0) {
    o[col] = 1.0f;
    if (a.amax) a.amax[(size_t)b * a.W + col] = 0;
    return;
  }
  if (a.readout == EWS_READOUT_MEAN) {
    float sum = 0.0f;
    for (int g2 = 0; g2 < RO_GROUPS; ++g2) sum += s_v[g2][cl];
    o[col] = sum / (float)a.n;
  } else {
    float best = s_v[0][cl];
    int bi = s_i[0][cl];
    for (int g2 = 1; g2 < RO_GROUPS; ++g2) {
      const int ti = s_i[g2][cl];
      if (ti < 0) continue;
      const float v = s_v[g2][cl];
      if (bi < 0 || v > best || (v == best && ti < bi)) {
        best = v;
        bi = ti;
      }
    }
    o[col] = best;
    if (a.amax) a.amax[(size_t)b * a.W + col] = bi;
  }
}

// ------------------------------------------------------------------------------------------------ backward
// adjoint scan LDS (floats): F, Ft, lambda2, S2 (state before the step), H, G1, G2 (32 x 36 each); vectors
constexpr int AD_F = 0, AD_FT = S32, AD_L2 = 2 * S32, AD_S2 = 3 * S32, AD_H = 4 * S32, AD_G1 = 5 * S32,
              AD_G2 = 6 * S32, AD_VEC = 7 * S32;  // lambda1, S1, s1, y1, rho1 (32 each)
constexpr int AD_FLOATS = AD_VEC + 5 * 32;
constexpr int ADJ_LOCAL = 0, ADJ_FULL = 1;

// one reverse step: (lambda1, lambda2) of the state after the step (row cotangent included) to the state before it;
// FULL: also ds1, ds2 (into dl) and dF (returned in the lane's tile entries) from the state before the step (S1, S2
// in LDS). The products run on MFMA over the first ku k-steps (every product has a factor that is zero past d in
// the summed index: a state, a cotangent or a product of one).
template <int N, int MODE>
__device__ __forceinline__ v4f adj_step(float* sm, float* dl, int ku) {
  float* F = sm + AD_F;
  float* Ft = sm + AD_FT;
  float* L2 = sm + AD_L2;
  float* S2 = sm + AD_S2;
  float* H = sm + AD_H;
  float* G1 = sm + AD_G1;
  float* G2 = sm + AD_G2;
  float* l1 = sm + AD_VEC;
  float* S1 = l1 + 32;
  float* s1 = l1 + 64;
  float* y1 = l1 + 96;
  float* rho = l1 + 128;
  const int i = (int)threadIdx.x >> 3;
  float r = 0.0f, y = 0.0f;
  if constexpr (N >= 2) {
    r = mv<false>(L2, s1);                                      // (lambda2 s1)[i]
    st_tile(H, mm_tile<false, false>(L2, F, zero4(), ku));      // H = lambda2 F
    if constexpr (MODE == ADJ_FULL) {
      y = mv<false>(F, S1);                                     // y1 = F S1
      st_tile(G1, mm_tile<false, false>(F, S2, zero4(), ku));   // G1 = F S2
      st_tile(G2, mm_tile<false, true>(F, S2, zero4(), ku));    // G2 = F S2^T
    }
  } else if constexpr (MODE == ADJ_FULL) {
    y = mv<false>(F, S1);
  }
  if (row_lead()) {
    rho[i] = l1[i] + r;
    y1[i] = y;
  }
  __syncthreads();
  v4f ln = zero4(), df = zero4();
  if constexpr (N >= 2) ln = mm_tile<false, false>(Ft, H, zero4(), ku);  // F^T H (Ft holds F^T row-major)
  const float l1n = mv<true>(F, rho);                                // (F^T rho)[i]
  if constexpr (MODE == ADJ_FULL) {
    float ds1 = l1[i];
    if constexpr (N >= 2) ds1 += mv<true>(L2, y1);  // lambda2^T y1
    if (row_lead()) dl[i] = ds1;
    // dF = rho S1^T + lambda2 G2 + lambda2^T G1
    if constexpr (N >= 2) {
      df = mm_tile<false, false>(L2, G2, df, ku);
      df = mm_tile<true, false>(L2, G1, df, ku);
      gst4(dl + DP, lds4(L2));  // ds2 = lambda2 (of the state after the step)
    }
    const int m = tile_m0() + 4 * tile_g(), n = tile_n0() + tile_i();
    const float sn = S1[n];
#pragma unroll
    for (int k = 0; k < 4; ++k) df[k] = fmaf(rho[m + k], sn, df[k]);
  }
  __syncthreads();
  if constexpr (N >= 2) st_tile(L2, ln);
  if (row_lead()) l1[i] = l1n;
  __syncthreads();
  return df;
}

template <int N, int MODE>
__global__ __launch_bounds__(NT) void k_wadj(WArgs a) {
  const int ku = (a.d + 3) >> 2;  // MFMA k-steps that reach a nonzero entry (d <= 4 ku)
  __shared__ __align__(16) float sm[AD_FLOATS];
  const int c = blockIdx.x, b = blockIdx.y;
  const int t0 = c * a.T, t1 = min(a.n, t0 + a.T);
  float* L2 = sm + AD_L2;
  float* l1 = sm + AD_VEC;
  float* S1 = l1 + 32;
  float* s1 = l1 + 64;
  float* S2 = sm + AD_S2;
  if (MODE == ADJ_LOCAL) {
    if (threadIdx.x < 32) l1[threadIdx.x] = 0.0f;
    sld4(L2, float4{0.0f, 0.0f, 0.0f, 0.0f});
  } else {
    load_state(a.lend + ((size_t)b * a.C + c) * RW, l1, L2);
  }
  const bool cached = a.flow_mode != EWS_FLOW_PER_INTERVAL;
  v4f dfs = zero4();  // shared-flow cotangent summed over the chunk's steps (the lane's tile entries)
  // The row cotangents come from the readout's cotangent (packed rows of W): the thread's level-1 entry (threads
  // below d) and its four level-2 entries (row i, columns j0 .. j0 + 3), zero in the padding. Prefix: row t of
  // gout; mean: gout / n at every step; terminal: gout at the last step; max: gout where the maximum's row is t.
  const int ri = trow<32>(), rj0 = tcol<32>(), d = a.d;
  const bool ok1 = (int)threadIdx.x < d;
  const int col1 = a.lvl0 + (int)threadIdx.x;
  bool ok2[4];
  int col2[4];
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    ok2[u] = N >= 2 && ri < d && rj0 + u < d;
    col2[u] = a.lvl0 + d + ri * d + rj0 + u;
  }
  float k1 = 0.0f, k2[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  int am1 = -1, am2[4] = {-1, -1, -1, -1};
  if (a.readout != EWS_READOUT_PREFIX) {  // one cotangent row per sample
    const float* g = a.gout + (size_t)b * a.W;
    if (ok1) k1 = a.readout == EWS_READOUT_MEAN ? g[col1] / (float)a.n : g[col1];
#pragma unroll
    for (int u = 0; u < 4; ++u)
      if (ok2[u]) k2[u] = a.readout == EWS_READOUT_MEAN ? g[col2[u]] / (float)a.n : g[col2[u]];
    if (a.readout == EWS_READOUT_MAX) {
      const int* am = a.amax + (size_t)b * a.W;
      if (ok1) am1 = am[col1];
#pragma unroll
      for (int u = 0; u < 4; ++u)
        if (ok2[u]) am2[u] = am[col2[u]];
    }
  }
  // the step's row cotangent, flow, s1 and (FULL) the state before it in registers, loaded during the step after
  float4 nF, ng2 = float4{0.0f, 0.0f, 0.0f, 0.0f}, nS2 = float4{0.0f, 0.0f, 0.0f, 0.0f};
  float ng1 = 0.0f, ns1 = 0.0f, nS1 = 0.0f;
  auto fetch = [&](int t) {
    const size_t r = (size_t)b * a.n + t;
    float c2[4];
    if (a.readout == EWS_READOUT_PREFIX) {
      const float* g = a.gout + r * a.W;
      ng1 = ok1 ? g[col1] : 0.0f;
#pragma unroll
      for (int u = 0; u < 4; ++u) c2[u] = ok2[u] ? g[col2[u]] : 0.0f;
    } else if (a.readout == EWS_READOUT_MEAN) {
      ng1 = k1;
#pragma unroll
      for (int u = 0; u < 4; ++u) c2[u] = k2[u];
    } else if (a.readout == EWS_READOUT_TERMINAL) {
      const bool last = t == a.n - 1;
      ng1 = last ? k1 : 0.0f;
#pragma unroll
      for (int u = 0; u < 4; ++u) c2[u] = last ? k2[u] : 0.0f;
    } else {
      ng1 = am1 == t ? k1 : 0.0f;
#pragma unroll
      for (int u = 0; u < 4; ++u) c2[u] = am2[u] == t ? k2[u] : 0.0f;
    }
    ng2 = float4{c2[0], c2[1], c2[2], c2[3]};
    if (threadIdx.x < 32) ns1 = a.loc[r * RW + threadIdx.x];
    nF = flow_regs(a, b, t);
    if (MODE == ADJ_FULL) {
      const float* sp = t > t0 ? a.rows + (r - 1) * RW : a.car + ((size_t)b * (a.C + 1) + c) * RW;
      if (threadIdx.x < 32) nS1 = sp[threadIdx.x];
      if (N >= 2) nS2 = gld4(sp + DP);
    }
  };
  fetch(t1 - 1);
  for (int t = t1 - 1; t >= t0; --t) {
    const size_t r = (size_t)b * a.n + t;
    if (threadIdx.x < 32) {
      l1[threadIdx.x] += ng1;
      s1[threadIdx.x] = ns1;
      if (MODE == ADJ_FULL) S1[threadIdx.x] = nS1;
    }
    if constexpr (N >= 2) {
      sld4(L2, f4add(lds4(L2), ng2));
      if (MODE == ADJ_FULL) sld4(S2, nS2);
    }
    commit_mat(nF, sm + AD_F, sm + AD_FT);
    __syncthreads();
    if (t > t0) fetch(t - 1);
    const v4f df = adj_step<N, MODE>(sm, MODE == ADJ_FULL ? a.dloc + r * RW : nullptr, ku);
    if constexpr (MODE == ADJ_FULL) {
      bool ident;
      flow_step(a, a.clock + (size_t)b * a.L, t, ident);
      if (!cached) {
        gst_tile(a.dfl + r * MM, df);
      } else if (!ident) {
        dfs += df;
      }
    }
  }
  if (MODE == ADJ_LOCAL) {
    store_state(a.mu + ((size_t)b * a.C + c) * RW, l1, L2);
  } else if (cached) {
    gst_tile(a.cpart + ((size_t)b * a.CP + c) * 3 * MM, dfs);
  }
}

// end cotangents of the chunks: lend[b][C-1] = 0, lend[b][c-1] = J_c^T lend[b][c] + mu[b][c] (J_c: chunk c's map)
template <int N>
__global__ __launch_bounds__(NT) void k_wadj_carry(WArgs a) {
  const int ku = (a.d + 3) >> 2;  // MFMA k-steps that reach a nonzero entry (d <= 4 ku)
  __shared__ __align__(16) float sm[AD_FLOATS];
  const int b = blockIdx.x;
  float* L2 = sm + AD_L2;
  float* l1 = sm + AD_VEC;
  float* s1 = l1 + 64;
  float* F = sm + AD_F;
  float* Ft = sm + AD_FT;
  if (threadIdx.x < 32) l1[threadIdx.x] = 0.0f;
  sld4(L2, float4{0.0f, 0.0f, 0.0f, 0.0f});
  __syncthreads();
  store_state(a.lend + ((size_t)b * a.C + a.C - 1) * RW, l1, L2);
  for (int c = a.C - 1; c >= 1; --c) {
    commit_mat(gld4(a.sfl + ((size_t)b * a.C + c) * MM), F, Ft);
    if (threadIdx.x < 32) s1[threadIdx.x] = a.summ[((size_t)b * a.C + c) * RW + threadIdx.x];
    __syncthreads();
    adj_step<N, ADJ_LOCAL>(sm, nullptr, ku);
    const float* m = a.mu + ((size_t)b * a.C + c) * RW;
    if (threadIdx.x < 32) l1[threadIdx.x] += m[threadIdx.x];
    if constexpr (N >= 2) sld4(L2, f4add(lds4(L2), gld4(m + DP)));
    __syncthreads();
    store_state(a.lend + ((size_t)b * a.C + c - 1) * RW, l1, L2);
  }
}

// Leaf adjoints, a workgroup per (slice of TL intervals, sample): dv per interval, the series leaf's dh and dA
// (workgroup partial), the Van Loan leaf's (dP, dV) per interval (per-interval mode) or summed over the slice (shared
// modes).
// LK: the leaf (LK_SERIES, LK_VL_SHARED, LK_VL_INT: the Van Loan leaf with shared or per-interval step matrices),
// one instantiation each so that each carries only its own registers
constexpr int LK_SERIES = 0, LK_VL_SHARED = 1, LK_VL_INT = 2;
template <int N, int LK>
__global__ __launch_bounds__(NT) void k_wleaf_bwd(WArgs a) {
  extern __shared__ __align__(16) float sm[];  // lf_floats(rows, 4) (+ LF_EXTRA, per-interval Van Loan)
  float* A = sm + LF_A;
  float* S2b = sm + LF_S2;  // ds2
  float* vec = sm + LF_VEC;
  float* ds1 = vec;
  float* wv = vec + 32;
  const int rows = a.leaf == EWS_LEAF_VAN_LOAN ? a.vm : a.q + 1;
  float* T1 = sm + LF_TAB;
  float* T2 = T1 + rows * 32;
  float* T3 = T2 + rows * 32;
  float* T4 = T3 + rows * 32;
  const int sl = blockIdx.x, b = blockIdx.y;
  const int t0 = sl * a.TL, t1 = min(a.n, t0 + a.TL);
  const int tid = threadIdx.x, i = tid >> 3, j0 = (tid & 7) * 4;
  load_A(a.d, a.A, A);
  float dA[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  float sP[4] = {0.0f, 0.0f, 0.0f, 0.0f}, sV[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  const float* th = a.clock + (size_t)b * a.L;
  constexpr bool vl = LK != LK_SERIES, vl_shared = LK == LK_VL_SHARED, vl_int = LK == LK_VL_INT;
  float* phi = sm + lf_floats(rows, 4);
  float* U = phi + LX_PHI;
  if (vl_int) {
    for (int e = tid; e < a.vm * (PW + 1); e += NT) phi[e] = a.apow[PHI_OFF + e];
  }
  // the interval's cotangents, increment and (per-interval Van Loan) step matrices in registers, loaded during the
  // interval before
  float nd1 = 0.0f, nv = 0.0f;
  float4 nd2 = float4{0.0f, 0.0f, 0.0f, 0.0f}, nP = nd2, nV = nd2;
  float nU[3] = {0.0f, 0.0f, 0.0f};  // (PW + 1) * 32 <= 3 NT
  bool nfixed = false;
  auto fetch = [&](int t) {
    const size_t r = (size_t)b * a.n + t;
    const float* x = a.path + ((size_t)b * a.L + t) * a.d;
    if (tid < 32) {
      nd1 = a.dloc[r * RW + tid];
      nv = tid < a.d ? x[a.d + tid] - x[tid] : 0.0f;
    }
    if (N >= 2) nd2 = gld4(a.dloc + r * RW + DP);
    if (vl_int && !(a.mflag[r] & 4)) {  // the series path: u_k, no (P, V)
      for (int k = 0; k < 3; ++k) {
        const int e = tid + k * NT;
        nU[k] = e < (PW + 1) * 32 ? a.ubuf[r * (PW + 1) * 32 + e] : 0.0f;
      }
    } else if (vl_int) {
      nP = gld4(a.vlm + r * 2 * MM);
      nV = gld4(a.vlm + r * 2 * MM + MM);
    } else if (vl_shared) {
      vl_step(a, th, t, nfixed);
      if (!nfixed) {
        nP = gld4(a.vlm + (size_t)b * 2 * MM);
        nV = gld4(a.vlm + (size_t)b * 2 * MM + MM);
      }
    }
  };
  if (t0 < t1) fetch(t0);
  __syncthreads();
  for (int t = t0; t < t1; ++t) {
    const size_t r = (size_t)b * a.n + t;
    if (tid < 32) {
      ds1[tid] = nd1;
      wv[tid] = vl ? nv / (float)a.vm : nv;
    }
    if constexpr (N >= 2) sld4(S2b, nd2);
    float dvi = 0.0f, dh = 0.0f;
    bool dv_done = false;  // dv of a series-path interval is k_wmat_bwd_series's
    if constexpr (vl) {
      float* P = sm + LF_P;
      float* V = sm + LF_V;
      const bool ser = vl_int && !(a.mflag[r] & 4);
      if (vl_shared && nfixed) {
        set_ident32(P, 1.0f);
        set_ident32(V, 1.0f);
      } else if (!ser) {
        sld4(P, nP);
        sld4(V, nV);
      } else {
        for (int k = 0; k < 3; ++k) {
          const int e = tid + k * NT;
          if (e < (PW + 1) * 32) U[e] = nU[k];
        }
      }
      const int M = a.vm;
      const float c = (th[t + 1] - th[t]) / (float)M;
      __syncthreads();
      if (t + 1 < t1) fetch(t + 1);
      if (ser) series_knots(M, phi, U, T1, c);  // Delta_m in rows 0 .. M-1
      else vl_knots(a, P, V, wv, T1);
      knot_sums(M, T1, T3, T2, nullptr);  // Z_m = R_m + Delta_m / 2 (T2), Y_m = Pre_m + Delta_m / 2 (T3)
      __syncthreads();
      // dDelta_m = ds1 + ds2 Z_m + ds2^T Y_m (rows of T4), a thread per entry
      for (int e = tid; e < M * 32; e += NT) {
        const int m = e >> 5, ii = e & 31;
        float v = ds1[ii];
        if constexpr (N >= 2) {
          const float* z = T2 + m * 32;
          const float* y = T3 + m * 32;
          const float* srow = S2b + ii * P32;
#pragma unroll 2
          for (int j = 0; j < 32; j += 4) {
            const float4 zz = *reinterpret_cast<const float4*>(z + j);
            const float4 yy = *reinterpret_cast<const float4*>(y + j);
            const float4 sr = *reinterpret_cast<const float4*>(srow + j);
            v = fmaf(sr.x, zz.x, v);
            v = fmaf(sr.y, zz.y, v);
            v = fmaf(sr.z, zz.z, v);
            v = fmaf(sr.w, zz.w, v);
            v = fmaf(S2b[j * P32 + ii], yy.x, v);
            v = fmaf(S2b[(j + 1) * P32 + ii], yy.y, v);
            v = fmaf(S2b[(j + 2) * P32 + ii], yy.z, v);
            v = fmaf(S2b[(j + 3) * P32 + ii], yy.w, v);
          }
        }
        T4[e] = v;
      }
      __syncthreads();
      if (ser) {
        // e_k = sum_r phi[r][k] dDelta_r, to ebuf: the powers' cotangent c^k e_k w^T, dw = sum_k c^k (A^k)^T e_k
        // and dc = sum_k k c^(k-1) <e_k, u_k> are k_wmat_bwd_series's (it holds the powers)
        for (int e = tid; e < (PW + 1) * 32; e += NT) {
          const int k = e >> 5, row = e & 31;
          float x = 0.0f;
          for (int m = 0; m < M; ++m) x = fmaf(phi[m * (PW + 1) + k], T4[m * 32 + row], x);
          a.ebuf[r * (PW + 1) * 32 + e] = x;
        }
        dv_done = true;
      } else {
      // chain: lam_1 = dDelta_1, lam_m = dDelta_m + P^T lam_{m-1} (in place in T4)
      for (int m = 1; m < M; ++m) {
        const float v = mv<true>(P, T4 + (m - 1) * 32);
        __syncthreads();
        if (row_lead()) T4[m * 32 + i] += v;
        __syncthreads();
      }
      // dP = sum_{m >= 1} lam_{m-1} Delta_m^T, dV = lam_M w^T, dv = V^T lam_M / M
      float gp[4] = {0.0f, 0.0f, 0.0f, 0.0f};
      for (int m = 1; m < M; ++m) {
        const float l = T4[(m - 1) * 32 + i];
        const float4 dm = *reinterpret_cast<const float4*>(T1 + m * 32 + j0);
        gp[0] = fmaf(l, dm.x, gp[0]);
        gp[1] = fmaf(l, dm.y, gp[1]);
        gp[2] = fmaf(l, dm.z, gp[2]);
        gp[3] = fmaf(l, dm.w, gp[3]);
      }
      const float lM = T4[(M - 1) * 32 + i];
      const float4 w4 = *reinterpret_cast<const float4*>(wv + j0);
      const float gv[4] = {lM * w4.x, lM * w4.y, lM * w4.z, lM * w4.w};
      dvi = mv<true>(V, T4 + (M - 1) * 32) / (float)M;
      bool fixed;
      vl_step(a, th, t, fixed);
      if (a.vl_mode == EWS_FLOW_PER_INTERVAL) {
        gst4(a.dvlm + r * 2 * MM, acc4(gp));
        gst4(a.dvlm + r * 2 * MM + MM, acc4(gv));
      } else if (!fixed) {
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          sP[k] += gp[k];
          sV[k] += gv[k];
        }
      }
      }
    } else {
      const int q = a.q;
      const float h = th[t + 1] - th[t];
      if (tid < 32) T1[tid] = wv[tid];
      __syncthreads();
      if (t + 1 < t1) fetch(t + 1);
      for (int p = 1; p <= q; ++p) {  // letters b_p (T1) and A b_{p-1} (T3)
        const float y = mv<false>(A, T1 + (p - 1) * 32);
        if (row_lead()) {
          T3[p * 32 + i] = y;
          T1[p * 32 + i] = (-h / (float)p) * y;
        }
        __syncthreads();
      }
      if constexpr (N >= 2) {  // u_p (T2) and w_p = sum_r C2[r][p] b_r (T4 for now)
        for (int e = tid; e < (q + 1) * 32; e += NT) {
          const int p = e >> 5, k = e & 31;
          float su = 0.0f, sw = 0.0f;
          for (int rr = 0; rr <= q - p; ++rr) {
            su = fmaf(c2coef(p, rr), T1[rr * 32 + k], su);
            sw = fmaf(c2coef(rr, p), T1[rr * 32 + k], sw);
          }
          T2[p * 32 + k] = su;
          T4[p * 32 + k] = sw;
        }
        __syncthreads();
      }
      // db_p = ds1 / (p + 1) + ds2 u_p + ds2^T w_p, kept by the row leads in registers: lane (i) of each p
      // goes through LDS: T4 row p is replaced by db_p
      for (int p = 0; p <= q; ++p) {
        float v = 0.0f;
        if constexpr (N >= 2) v = mv<false>(S2b, T2 + p * 32) + mv<true>(S2b, T4 + p * 32);
        __syncthreads();
        if (row_lead()) T4[p * 32 + i] = fmaf(inv_f(p + 1), ds1[i], v);
        __syncthreads();
      }
      // reverse recursion: for p = q .. 1: dh += -(1/p) <db_p, A b_{p-1}>, dA += (-h/p) db_p b_{p-1}^T,
      // db_{p-1} += (-h/p) A^T db_p
      for (int p = q; p >= 1; --p) {
        const float cpf = -h / (float)p;
        const float dbi = T4[p * 32 + i];
        const float4 bp = *reinterpret_cast<const float4*>(T1 + (p - 1) * 32 + j0);
        dA[0] = fmaf(cpf * dbi, bp.x, dA[0]);
        dA[1] = fmaf(cpf * dbi, bp.y, dA[1]);
        dA[2] = fmaf(cpf * dbi, bp.z, dA[2]);
        dA[3] = fmaf(cpf * dbi, bp.w, dA[3]);
        if (tid < 32) dh = fmaf(-inv_f(p) * T4[p * 32 + tid], T3[p * 32 + tid], dh);
        const float v = mv<true>(A, T4 + p * 32);
        __syncthreads();
        if (row_lead()) T4[(p - 1) * 32 + i] = fmaf(cpf, v, T4[(p - 1) * 32 + i]);
        __syncthreads();
      }
      dvi = T4[i];
    }
    if (!dv_done && row_lead() && i < a.d) a.dv[r * DP + i] = dvi;
    if constexpr (!vl) {
      // dh: the 32 partials of threads 0..31 (wavefront 0)
      float s = tid < 32 ? dh : 0.0f;
      if (tid < 64) {
        s = lanes::sum_n(s, 32);
        if (tid == 0) a.dhl[r] = s;
      }
    }
    __syncthreads();
  }
  if (vl_shared) {
    float* cp = a.cpart + ((size_t)b * a.CP + sl) * 3 * MM;
    gst4(cp + MM, acc4(sP));
    gst4(cp + 2 * MM, acc4(sV));
  }
  if constexpr (!vl) gst4(a.apart + ((size_t)b * a.NSL + sl) * MM, acc4(dA));  // (the Van Loan leaf has none)
}

// ------------------------------------------------------------------------------------------------ slice leaf
// The Van Loan leaf with the shared pair (uniform reweighting modes) and M <= VLS_M knots, a workgroup per slice of
// VLS_T consecutive intervals of one sample: (P, V) is the same for every interval of the sample, so the knots of
// the whole slice are products of 32 x 32 matrices with 32 x VLS_T blocks (one column per interval), the knots'
// adjoint chain likewise, and the pair's cotangent sums over the slice are products over its intervals: a barrier
// per product for the slice instead of one per matrix-vector product per interval. A step the mode fixes to the
// identity (the basepoint interval) takes P = V = I: its column is patched after each product.
constexpr int VLS_M = 4, VLS_T = 16, VLS_B = 32 * VLS_T;  // knots at most, intervals per slice, floats per block
// LDS (floats) of the forward: P, V, W (the slice's w = v / M), knots D (VLS_M blocks), Y (VLS_M blocks)
constexpr int VF_P = 0, VF_V = S32, VF_W = 2 * S32, VF_D = VF_W + VLS_B, VF_Y = VF_D + VLS_M * VLS_B,
              VF_FLOATS = VF_Y + VLS_M * VLS_B;
// of the backward: the same, then DD (the knots' cotangents), the cotangent staging of two intervals (ds2), the
// slice's ds1 and s1 (S, the knots' sums); Y becomes the chain's lambda once DD is formed
constexpr int VB_DD = VF_FLOATS, VB_G2 = VB_DD + VLS_M * VLS_B, VB_G1 = VB_G2 + 2 * S32, VB_S = VB_G1 + VLS_B,
              VB_MASK = VB_S + VLS_B, VB_FLOATS = VB_MASK + VLS_T;

// Z[r][t] = sum_k Mx(r, k) X[k][t] for the thread's row r = tid / 8 and columns t, t + 1 (t = 2 (tid % 8));
// Mx(r, k) = Mx[k][r] when TM; Mx at pitch 36, X and Z blocks of 32 x VLS_T
template <bool TM>
__device__ __forceinline__ float2 mcols(const float* Mx, const float* X) {
  const int r = (int)threadIdx.x >> 3, t = ((int)threadIdx.x & 7) * 2;
  float2 acc = float2{0.0f, 0.0f};
#pragma unroll 8
  for (int k = 0; k < 32; ++k) {
    const float m = TM ? Mx[k * P32 + r] : Mx[r * P32 + k];
    const float2 x = *reinterpret_cast<const float2*>(X + k * VLS_T + t);
    acc.x = fmaf(m, x.x, acc.x);
    acc.y = fmaf(m, x.y, acc.y);
  }
  return acc;
}

// the slice's P, V (identity when the mode fixes every step), W and the fixed-column mask; returns the slice's
// interval count
__device__ int vls_stage(const WArgs& a, float* sm, int b, int t0, int t1, float* mask) {
  const float* th = a.clock + (size_t)b * a.L;
  bool all_fixed;
  vl_step(a, th, 1, all_fixed);  // a zero shared step: every interval's pair is the identity
  float* P = sm + VF_P;
  float* V = sm + VF_V;
  if (all_fixed) {
    set_ident32(P, 1.0f);
    set_ident32(V, 1.0f);
  } else {
    sld4(P, gld4(a.vlm + (size_t)b * 2 * MM));
    sld4(V, gld4(a.vlm + (size_t)b * 2 * MM + MM));
  }
  const int nt = t1 - t0;
  for (int e = threadIdx.x; e < VLS_B; e += NT) {  // W[k][t]
    const int k = e / VLS_T, t = e - k * VLS_T;
    float w = 0.0f;
    if (t < nt && k < a.d) {
      const float* x = a.path + ((size_t)b * a.L + t0 + t) * a.d;
      w = (x[a.d + k] - x[k]) / (float)a.vm;
    }
    sm[VF_W + e] = w;
  }
  if (mask && threadIdx.x < VLS_T) {  // 1: the pair's cotangent gets this interval's terms
    bool fixed = true;
    if ((int)threadIdx.x < nt) vl_step(a, th, t0 + threadIdx.x, fixed);
    mask[threadIdx.x] = fixed ? 0.0f : 1.0f;
  }
  return nt;
}

// knots of the slice: D_{M-1} = V W, D_{m-1} = P D_m (block m - 1 holds Delta_m); a fixed column keeps w
__device__ void vls_knots(const WArgs& a, float* sm, int t0) {
  const int M = a.vm, r = (int)threadIdx.x >> 3, t = ((int)threadIdx.x & 7) * 2;
  const bool fix0 = a.vl_mode == EWS_FLOW_CACHED_BASEPOINT && t0 == 0;  // the basepoint interval: P = V = I
  float* D = sm + VF_D;
  const float* W = sm + VF_W;
  __syncthreads();
  float2 y = mcols<false>(sm + VF_V, W);
  if (fix0 && t == 0) y.x = W[r * VLS_T];
  *reinterpret_cast<float2*>(D + (M - 1) * VLS_B + r * VLS_T + t) = y;
  __syncthreads();
  for (int m = M - 1; m >= 1; --m) {
    y = mcols<false>(sm + VF_P, D + m * VLS_B);
    if (fix0 && t == 0) y.x = D[m * VLS_B + r * VLS_T];
    *reinterpret_cast<float2*>(D + (m - 1) * VLS_B + r * VLS_T + t) = y;
    __syncthreads();
  }
}

// Y_m = Pre_m + Delta_m / 2 per (row, column) (thread: row tid / 8, columns 2 (tid % 8) .. + 1); returns the
// columns' sums s1
__device__ float2 vls_sums(int M, float* sm) {
  const int r = (int)threadIdx.x >> 3, t = ((int)threadIdx.x & 7) * 2;
  const float* D = sm + VF_D;
  float* Y = sm + VF_Y;
  float2 pre = float2{0.0f, 0.0f};
  for (int m = 0; m < M; ++m) {
    const float2 dm = *reinterpret_cast<const float2*>(D + m * VLS_B + r * VLS_T + t);
    *reinterpret_cast<float2*>(Y + m * VLS_B + r * VLS_T + t) =
        float2{fmaf(0.5f, dm.x, pre.x), fmaf(0.5f, dm.y, pre.y)};
    pre.x += dm.x;
    pre.y += dm.y;
  }
  return pre;
}

template <int N>
__global__ __launch_bounds__(NT) void k_wleaf_vls(WArgs a) {
  extern __shared__ __align__(16) float sm[];  // VF_FLOATS
  const int sl = blockIdx.x, b = blockIdx.y, t0 = sl * VLS_T, t1 = min(a.n, t0 + VLS_T), M = a.vm;
  const int nt = vls_stage(a, sm, b, t0, t1, nullptr);
  vls_knots(a, sm, t0);
  const float2 s1 = vls_sums(M, sm);
  const int r = (int)threadIdx.x >> 3, tc = ((int)threadIdx.x & 7) * 2;
  if (tc < nt) a.loc[((size_t)b * a.n + t0 + tc) * RW + r] = s1.x;
  if (tc + 1 < nt) a.loc[((size_t)b * a.n + t0 + tc + 1) * RW + r] = s1.y;
  if constexpr (N >= 2) {  // s2_t = sum_m Y_m Delta_m^T per interval: one MFMA tile per wavefront, K = the knots
    __syncthreads();
    const float* D = sm + VF_D;
    const float* Y = sm + VF_Y;
    const int m0 = tile_m0(), n0 = tile_n0(), ti = tile_i(), g = tile_g();  // g: the knot (K index)
    for (int t = 0; t < nt; ++t) {
      const float ya = g < M ? Y[g * VLS_B + (m0 + ti) * VLS_T + t] : 0.0f;
      const float db = g < M ? D[g * VLS_B + (n0 + ti) * VLS_T + t] : 0.0f;
      const v4f s2 = __builtin_amdgcn_mfma_f32_16x16x4f32(ya, db, zero4(), 0, 0, 0);
      gst_tile(a.loc + ((size_t)b * a.n + t0 + t) * RW + DP, s2);
    }
  }
}

// Adjoint of the slice leaf: dDelta_m = ds1 + ds2 (S - Y_m) + ds2^T Y_m per interval (two intervals at a time:
// Z_m = S - Y_m, S the interval's s1), then the chain lambda_0 = dD_0, lambda_m = dD_m + P^T lambda_{m-1} for the
// slice, dP = sum_{m >= 1} lambda_{m-1} D_m^T and dV = lambda_{M-1} W^T over its non-fixed intervals (into cpart),
// dv = V^T lambda_{M-1} / M
template <int N>
__global__ __launch_bounds__(NT) void k_wleaf_bwd_vls(WArgs a) {
  extern __shared__ __align__(16) float sm[];  // VB_FLOATS
  const int sl = blockIdx.x, b = blockIdx.y, t0 = sl * VLS_T, t1 = min(a.n, t0 + VLS_T), M = a.vm;
  const int tid = threadIdx.x;
  float* mask = sm + VB_MASK;
  float* DD = sm + VB_DD;
  float* G2 = sm + VB_G2;
  float* G1 = sm + VB_G1;  // ds1 of the slice, G1[t][k]
  // the slice's ds1 and the first two intervals' ds2, loaded ahead of the knots
  const int nt = vls_stage(a, sm, b, t0, t1, mask);
  for (int e = tid; e < VLS_B; e += NT) {
    const int t = e >> 5, k = e & 31;
    G1[e] = t < nt ? a.dloc[((size_t)b * a.n + t0 + t) * RW + k] : 0.0f;
  }
  float4 nd2[2] = {float4{0.0f, 0.0f, 0.0f, 0.0f}, float4{0.0f, 0.0f, 0.0f, 0.0f}};
  auto fetch = [&](int tp) {
#pragma unroll
    for (int u = 0; u < 2; ++u)
      if (N >= 2 && tp + u < nt) nd2[u] = gld4(a.dloc + ((size_t)b * a.n + t0 + tp + u) * RW + DP);
  };
  fetch(0);
  for (int e = tid; e < VLS_M * VLS_B; e += NT) DD[e] = 0.0f;  // the columns past the slice's end stay zero
  vls_knots(a, sm, t0);
  {
    const float2 s1 = vls_sums(M, sm);
    *reinterpret_cast<float2*>(sm + VB_S + (tid >> 3) * VLS_T + (tid & 7) * 2) = s1;
  }
  // dD for two intervals at a time: thread (u = tid / 128, m = (tid / 32) % 4, row = tid % 32)
  const int u = tid >> 7, mm = (tid >> 5) & 3, row = tid & 31;
  const float* Y = sm + VF_Y;
  const float* D = sm + VF_D;
  for (int tp = 0; tp < nt; tp += 2) {
    if constexpr (N >= 2) {
      sld4(G2, nd2[0]);
      sld4(G2 + S32, nd2[1]);
    }
    __syncthreads();
    if (tp + 2 < nt) fetch(tp + 2);
    const int t = tp + u;
    if (mm < M && t < nt) {
      float v = G1[t * 32 + row];
      if constexpr (N >= 2) {
        const float* g2 = G2 + u * S32;
        const float* y = Y + mm * VLS_B + t;
        const float* sv = sm + VB_S + t;
        float sz = 0.0f, sy = 0.0f;  // (ds2 Z_m)[row], (ds2^T Y_m)[row]
#pragma unroll 8
        for (int k = 0; k < 32; ++k) {
          const float yk = y[k * VLS_T];
          sz = fmaf(g2[row * P32 + k], sv[k * VLS_T] - yk, sz);
          sy = fmaf(g2[k * P32 + row], yk, sy);
        }
        v += sz + sy;
      }
      DD[mm * VLS_B + row * VLS_T + t] = v;
    }
    __syncthreads();
  }
  // the chain over the slice (Y's blocks become lambda): L_0 = DD_0, L_m = DD_m + P^T L_{m-1}; a fixed column
  // (P = I) adds L_{m-1} itself
  float* L = sm + VF_Y;
  const int r = tid >> 3, tc = (tid & 7) * 2;
  const bool fix0 = a.vl_mode == EWS_FLOW_CACHED_BASEPOINT && t0 == 0;
  *reinterpret_cast<float2*>(L + r * VLS_T + tc) = *reinterpret_cast<const float2*>(DD + r * VLS_T + tc);
  __syncthreads();
  for (int m = 1; m < M; ++m) {
    float2 y2 = mcols<true>(sm + VF_P, L + (m - 1) * VLS_B);
    if (fix0 && tc == 0) y2.x = L[(m - 1) * VLS_B + r * VLS_T];
    const float2 dd = *reinterpret_cast<const float2*>(DD + m * VLS_B + r * VLS_T + tc);
    *reinterpret_cast<float2*>(L + m * VLS_B + r * VLS_T + tc) = float2{dd.x + y2.x, dd.y + y2.y};
    __syncthreads();
  }
  // dv = V^T L_{M-1} / M (a fixed column: L_{M-1} / M)
  {
    float2 y2 = mcols<true>(sm + VF_V, L + (M - 1) * VLS_B);
    if (fix0 && tc == 0) y2.x = L[(M - 1) * VLS_B + r * VLS_T];
    if (r < a.d) {
      if (tc < nt) a.dv[((size_t)b * a.n + t0 + tc) * DP + r] = y2.x / (float)M;
      if (tc + 1 < nt) a.dv[((size_t)b * a.n + t0 + tc + 1) * DP + r] = y2.y / (float)M;
    }
  }
  // dP = sum_{m >= 1} L_{m-1} D_m^T, dV = L_{M-1} W^T over the non-fixed intervals: products over the slice's
  // columns (K = VLS_T, four k-steps) on MFMA, the wavefront's tile of each
  const float* W = sm + VF_W;
  const int m0 = tile_m0(), n0 = tile_n0(), ti = tile_i(), g = tile_g();
  v4f gp = zero4(), gv = zero4();
#pragma unroll
  for (int uu = 0; uu < VLS_T / 4; ++uu) {
    const int t = 4 * uu + g;
    const float mk = mask[t];
    for (int m = 1; m < M; ++m)
      gp = __builtin_amdgcn_mfma_f32_16x16x4f32(mk * L[(m - 1) * VLS_B + (m0 + ti) * VLS_T + t],
                                               D[m * VLS_B + (n0 + ti) * VLS_T + t], gp, 0, 0, 0);
    gv = __builtin_amdgcn_mfma_f32_16x16x4f32(mk * L[(M - 1) * VLS_B + (m0 + ti) * VLS_T + t],
                                             W[(n0 + ti) * VLS_T + t], gv, 0, 0, 0);
  }
  float* cp = a.cpart + ((size_t)b * a.CP + sl) * 3 * MM;
  gst_tile(cp + MM, gp);
  gst_tile(cp + 2 * MM, gv);
}

// Matrix-function adjoints. per_interval: one item per interval, the flow's (dfl) and the Van Loan pair's (dvlm)
// cotangents of the per-interval modes, dh into dhm (flow, Van Loan); else one item per sample, the partials of the
// shared flow (per chunk) and pair (per leaf slice) summed in order, the shared steps' gradients into dsh[b][0..1].
// dA: workgroup partials at apart + slot0 (grid row by row).
__global__ __launch_bounds__(NT) void k_wmat_bwd(WArgs a, int mode, long slot0) {
  extern __shared__ __align__(16) float sm[];
  float* A = sm + MF_A;
  load_A(a.d, a.A, A);
  __syncthreads();
  float dA[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  const int per_interval = mode != 0;
  const long items = per_interval ? (long)a.B * a.n : a.B;
  // with two grid rows, row 0 takes the flows and row 1 the Van Loan pairs
  const bool do_flow = (a.flow_mode == EWS_FLOW_PER_INTERVAL) == (per_interval != 0) &&
                       (gridDim.y == 1 || blockIdx.y == 0);
  const bool do_vl = a.leaf == EWS_LEAF_VAN_LOAN && (a.vl_mode == EWS_FLOW_PER_INTERVAL) == (per_interval != 0) &&
                     (gridDim.y == 1 || blockIdx.y == 1);
  float* G0 = sm + MF_T;
  float* G1 = sm + MF_U;
  const int need = (do_flow ? 1 : 0) | (do_vl ? 2 : 0);
  for (long it = next_item(a, mode, need, -1, items), it_end = item_end(mode, items); it < it_end;
       it = next_item(a, mode, need, it, items)) {
    const int b = per_interval ? (int)(it / a.n) : (int)it;
    const int t = per_interval ? (int)(it - (long)b * a.n) : 1;
    const float* th = a.clock + (size_t)b * a.L;
    float dh_f = 0.0f, dh_v = 0.0f;
    const int flag = mode == 2 ? a.mflag[it] : a.sflag[it];  // the matrices outside the series radius
    const bool run_f = do_flow && (flag & 1), run_v = do_vl && (flag & 2);
    if (run_f) {
      bool ident;
      const float h = flow_step(a, th, t, ident);
      float g[4];
      if (per_interval) {
        const float4 v = gld4(a.dfl + it * MM);
        g[0] = v.x; g[1] = v.y; g[2] = v.z; g[3] = v.w;
      } else {
        g[0] = g[1] = g[2] = g[3] = 0.0f;
        for (int c = 0; c < a.C; ++c) {
          const float4 v = gld4(a.cpart + ((size_t)b * a.CP + c) * 3 * MM);
          g[0] += v.x; g[1] += v.y; g[2] += v.z; g[3] += v.w;
        }
      }
      __syncthreads();
      st<32>(G0, g);
      __syncthreads();
      float xb[4];
      matfn_bwd(sm, a.chen, true, h, xb);
      const float4 av = lds4(A);
      const float dot = xb[0] * av.x + xb[1] * av.y + xb[2] * av.z + xb[3] * av.w;
#pragma unroll
      for (int k = 0; k < 4; ++k) dA[k] = fmaf(h, xb[k], dA[k]);
      dh_f = block_sum(dot, sm + MF_RED);
    }
    if (run_v) {
      bool fixed;
      const float cst = vl_step(a, th, t, fixed);
      if (!fixed) {
        float g0[4], g1[4];
        if (per_interval) {
          const float4 p = gld4(a.dvlm + it * 2 * MM), v = gld4(a.dvlm + it * 2 * MM + MM);
          g0[0] = p.x; g0[1] = p.y; g0[2] = p.z; g0[3] = p.w;
          g1[0] = v.x; g1[1] = v.y; g1[2] = v.z; g1[3] = v.w;
        } else {
#pragma unroll
          for (int k = 0; k < 4; ++k) g0[k] = g1[k] = 0.0f;
          for (int c = 0; c < a.NSL; ++c) {
            const float* cp = a.cpart + ((size_t)b * a.CP + c) * 3 * MM;
            const float4 p = gld4(cp + MM), v = gld4(cp + 2 * MM);
            g0[0] += p.x; g0[1] += p.y; g0[2] += p.z; g0[3] += p.w;
            g1[0] += v.x; g1[1] += v.y; g1[2] += v.z; g1[3] += v.w;
          }
        }
        __syncthreads();
        st<32>(G0, g0);
        st<32>(G1, g1);
        __syncthreads();
        float xb[4];
        matfn_bwd(sm, a.vl_expm, false, cst, xb);
        const float4 av = lds4(A);
        const float dot = xb[0] * av.x + xb[1] * av.y + xb[2] * av.z + xb[3] * av.w;
#pragma unroll
        for (int k = 0; k < 4; ++k) dA[k] = fmaf(cst, xb[k], dA[k]);
        dh_v = block_sum(dot, sm + MF_RED) / (float)a.vm;  // c = dt / M
      }
    }
    if (threadIdx.x == 0) {  // [flow, Van Loan] per interval or per sample
      float* dst = per_interval ? a.dhm + 2 * it : a.dsh + 2 * b;
      if (run_f) dst[0] = dh_f;
      if (run_v) dst[1] = dh_v;
    }
    __syncthreads();
  }
  gst4(a.apart + (slot0 + (long)blockIdx.y * gridDim.x + blockIdx.x) * MM, acc4(dA));
}

// grad_A = sum of the partials first .. nparts - 1 (float64; the Van Loan leaf's adjoint writes none, so its slots
// are skipped): a workgroup per 16 entries, 16 interleaved groups of slots combined in a fixed order; entries i, j < d
__global__ __launch_bounds__(NT) void k_wfinal_A(WArgs a, long first, long nparts, float* grad_A) {
  __shared__ double s_p[16][16];
  const int el = threadIdx.x & 15, grp = threadIdx.x >> 4;
  const int e = blockIdx.x * 16 + el;
  double s = 0.0;
  for (long k = first + grp; k < nparts; k += 16) s += (double)a.apart[k * MM + e];
  s_p[grp][el] = s;
  __syncthreads();
  if (grp != 0) return;
  double tot = 0.0;
  for (int g2 = 0; g2 < 16; ++g2) tot += s_p[g2][el];
  const int r = e >> 5, c = e & 31;
  if (r < a.d && c < a.d) grad_A[r * a.d + c] = (float)tot;
}

// grad_path[b][k] = dv[k-1] - dv[k]; grad_clock[b][k] = dh[k-1] - dh[k] plus the shared steps' gradients
__global__ __launch_bounds__(NT) void k_wknots(WArgs a, float* grad_path, float* grad_clock) {
  const int b = blockIdx.y;
  const int k = blockIdx.x * NT + threadIdx.x;
  if (k >= a.L) return;
  const size_t base = (size_t)b * a.n;
  for (int ch = 0; ch < a.d; ++ch) {
    const float lo = k >= 1 ? a.dv[(base + k - 1) * DP + ch] : 0.0f;
    const float hi = k < a.n ? a.dv[(base + k) * DP + ch] : 0.0f;
    grad_path[((size_t)b * a.L + k) * a.d + ch] = lo - hi;
  }
  if (!grad_clock) return;
  auto dh = [&](int t) -> float {
    float s = 0.0f;
    if (a.leaf != EWS_LEAF_VAN_LOAN) s += a.dhl[base + t];
    if (a.flow_mode == EWS_FLOW_PER_INTERVAL) s += a.dhm[2 * (base + t)];
    if (a.leaf == EWS_LEAF_VAN_LOAN && a.vl_mode == EWS_FLOW_PER_INTERVAL) s += a.dhm[2 * (base + t) + 1];
    return s;
  };
  float g = (k >= 1 ? dh(k - 1) : 0.0f) - (k < a.n ? dh(k) : 0.0f);
  // shared steps: th[1] - th[0] (uniform) or th[2] - th[1] (basepoint)
  if (a.flow_mode != EWS_FLOW_PER_INTERVAL) {
    const int k0 = a.flow_mode == EWS_FLOW_CACHED ? 0 : 1;
    if (k == k0) g -= a.dsh[2 * b];
    if (k == k0 + 1) g += a.dsh[2 * b];
  }
  if (a.leaf == EWS_LEAF_VAN_LOAN && a.vl_mode != EWS_FLOW_PER_INTERVAL) {
    const int k0 = a.vl_mode == EWS_FLOW_CACHED ? 0 : 1;
    if (k == k0) g -= a.dsh[2 * b + 1];
    if (k == k0 + 1) g += a.dsh[2 * b + 1];
  }
  grad_clock[(size_t)b * a.L + k] = g;
}

}  // namespace wide
}  // namespace ews

// ------------------------------------------------------------------------------------------------ host side
namespace ews {
namespace wide {
namespace {

size_t al256(size_t x) { return (x + 255) & ~(size_t)255; }

constexpr int kLeafSlice = 16;  // intervals per workgroup of the leaf adjoint

struct WPlan {
  int B, L, n, d, N, T, C, W, TL, NSL, CP, rows;  // rows: knots M or letters q + 1 of the leaf tables
  bool fl_int, vl, vl_int, vls, exact_int, exact_smp, mats_int, mats_smp;
  long g_int, g_smp;   // workgroups of the matrix-function adjoints (per grid row; per interval: the flagged ones)
  long g_ser;          // workgroups of the series path's adjoint
  int gy_int, gy_smp;  // grid rows: 2 when both the flows and the Van Loan pairs are of that kind
};

int plan(const ews_dense_desc* s, WPlan& p) {
  if (!s) return EWS_ERR_NULL;
  if (s->depth < 1 || s->depth > 2) return EWS_ERR_DEPTH;
  if (s->batch < 1 || s->length < 2 || s->dim <= 16 || s->dim > DP) return EWS_ERR_SHAPE;
  if (s->flow_mode < 0 || s->flow_mode > 2 || s->readout < 0 || s->readout > 3) return EWS_ERR_OPTION;
  if (s->leaf != EWS_LEAF_SERIES && s->leaf != EWS_LEAF_VAN_LOAN) return EWS_ERR_OPTION;
  const bool vl = s->leaf == EWS_LEAF_VAN_LOAN;
  if (!vl && (s->series_q < 0 || s->series_q > QMAXW)) return EWS_ERR_OPTION;
  if (vl && (s->vl_steps < 1 || s->vl_steps > VMAXK)) return EWS_ERR_OPTION;
  if (vl && (s->vl_expm < 0 || s->vl_expm > 3 || s->vl_mode < 0 || s->vl_mode > 2)) return EWS_ERR_OPTION;
  if (s->chen_expm < 0 || s->chen_expm > 3) return EWS_ERR_OPTION;
  if (s->flow_mode == EWS_FLOW_CACHED_BASEPOINT && s->length < 3) return EWS_ERR_SHAPE;
  if (vl && s->vl_mode == EWS_FLOW_CACHED_BASEPOINT && s->length < 3) return EWS_ERR_SHAPE;
  if (s->chunk < 0) return EWS_ERR_SHAPE;
  p.B = s->batch;
  p.L = s->length;
  p.n = p.L - 1;
  p.d = s->dim;
  p.N = s->depth;
  // default chunk: 64 intervals, or 32 when that leaves fewer than two chunk workgroups per CU (measured at
  // B = 32, L = 896: 32 takes 3-4% less time than 64, 16 and 48 none)
  p.T = s->chunk ? s->chunk : ((long)s->batch * ((s->length - 1 + 63) / 64) < 512 ? 32 : 64);
  p.C = (p.n + p.T - 1) / p.T;
  p.TL = kLeafSlice;
  p.NSL = (p.n + p.TL - 1) / p.TL;
  p.CP = std::max(p.C, p.NSL);
  p.W = p.d + (p.N >= 2 ? p.d * p.d : 0) + (s->level0 ? 1 : 0);
  p.fl_int = s->flow_mode == EWS_FLOW_PER_INTERVAL;
  p.vl = vl;
  p.rows = vl ? s->vl_steps : s->series_q + 1;
  p.vl_int = vl && s->vl_mode == EWS_FLOW_PER_INTERVAL;
  static_assert(kLeafSlice == VLS_T, "the slice leaf kernels take the leaf adjoint's slices");
  p.vls = vl && !p.vl_int && s->vl_steps <= VLS_M;  // the shared pair with few knots: slice leaf kernels
  p.mats_int = p.fl_int || p.vl_int;
  p.mats_smp = !p.fl_int || (vl && !p.vl_int);
  p.exact_int = (p.fl_int && s->chen_expm == EWS_EXPM_EXACT) || (p.vl_int && s->vl_expm == EWS_EXPM_EXACT);
  p.exact_smp = (!p.fl_int && s->chen_expm == EWS_EXPM_EXACT) || (vl && !p.vl_int && s->vl_expm == EWS_EXPM_EXACT);
  p.g_int = p.mats_int ? std::min<long>((long)p.B * p.n, 256) : 0;
  p.g_ser = p.mats_int ? std::min<long>((long)p.B * p.n, 512) : 0;  // two workgroups per CU
  p.g_smp = p.mats_smp ? p.B : 0;
  p.gy_int = p.fl_int && p.vl_int ? 2 : 1;
  p.gy_smp = !p.fl_int && vl && !p.vl_int ? 2 : 1;
  return EWS_OK;
}

struct WLay {
  size_t fl, vlm, loc, summ, sfl, car, rows, rpart, ridx, amax, apow, mflag, sflag, outs, mu, lend, dloc, dfl, cpart,
      dvlm, apart, dv, dhl, dhm, dsh, hpart, hsum, ubuf, ebuf, total;
};

WLay layout(const ews_dense_desc* s, const WPlan& p, bool bwd) {
  WLay w{};
  size_t off = 0;
  const size_t BN = (size_t)p.B * p.n, BC = (size_t)p.B * p.C;
  auto take = [&](size_t& f, size_t bytes) {
    f = off;
    off += al256(bytes);
  };
  take(w.fl, (p.fl_int ? BN : (size_t)p.B) * MM * 4);
  take(w.vlm, p.vl ? (p.vl_int ? BN : (size_t)p.B) * 2 * MM * 4 : 0);
  take(w.loc, BN * RW * 4);
  take(w.summ, BC * RW * 4);
  take(w.sfl, BC * MM * 4);
  take(w.car, (size_t)p.B * (p.C + 1) * RW * 4);
  const bool mm_ro = s->readout == EWS_READOUT_MEAN || s->readout == EWS_READOUT_MAX;
  take(w.rows, bwd ? BN * RW * 4 : 0);
  take(w.rpart, mm_ro ? BC * RW * 4 : 0);
  take(w.ridx, s->readout == EWS_READOUT_MAX ? BC * RW * 4 : 0);
  take(w.amax, s->readout == EWS_READOUT_MAX ? (size_t)p.B * p.W * 4 : 0);
  take(w.apow, (size_t)APOW_FLOATS * 4);  // the series path serves both per-interval and per-sample matrices
  take(w.mflag, p.mats_int ? BN * 4 : 0);
  take(w.sflag, p.mats_smp ? (size_t)p.B * 4 : 0);
  take(w.ubuf, p.vl_int ? BN * (PW + 1) * 32 * 4 : 0);
  if (bwd) {
    take(w.outs, s->readout == EWS_READOUT_MAX ? (size_t)p.B * p.W * 4 : 0);
    take(w.mu, BC * RW * 4);
    take(w.lend, BC * RW * 4);
    take(w.dloc, BN * RW * 4);
    take(w.dfl, p.fl_int ? BN * MM * 4 : 0);
    take(w.cpart, (size_t)p.B * p.CP * 3 * MM * 4);
    take(w.dvlm, p.vl_int ? BN * 2 * MM * 4 : 0);
    take(w.apart, ((size_t)p.B * p.NSL + p.g_int * p.gy_int + p.g_smp * p.gy_smp + 1) * MM * 4);
    take(w.dv, BN * DP * 4);
    take(w.dhl, BN * 4);
    take(w.dhm, BN * 2 * 4);
    take(w.dsh, (size_t)p.B * 2 * 4);
    take(w.hpart, (size_t)(p.g_ser + (p.mats_smp ? p.B : 0)) * (PW + 1) * MM * 4);
    take(w.hsum, (size_t)(PW + 1) * MM * 8);
    take(w.ebuf, p.vl_int ? BN * (PW + 1) * 32 * 4 : 0);
  }
  w.total = off;
  return w;
}

WArgs make_args(const ews_dense_desc* s, const WPlan& p, const float* path, const float* clock, const float* A,
                float* out, void* workspace, bool bwd) {
  WArgs a{};
  a.B = p.B; a.L = p.L; a.n = p.n; a.d = p.d; a.N = p.N; a.T = p.T; a.C = p.C; a.W = p.W;
  a.TL = p.TL; a.NSL = p.NSL; a.CP = p.CP;
  a.lvl0 = s->level0 ? 1 : 0; a.readout = s->readout;
  a.flow_mode = s->flow_mode; a.chen = s->chen_expm; a.leaf = s->leaf;
  a.q = p.vl ? 0 : s->series_q; a.vm = p.vl ? s->vl_steps : 0;
  a.vl_expm = p.vl ? s->vl_expm : 0; a.vl_mode = p.vl ? s->vl_mode : 0;
  a.path = path; a.clock = clock; a.A = A; a.out = out;
  const WLay w = layout(s, p, bwd);
  char* ws = (char*)workspace;
  auto f = [&](size_t o) { return (float*)(ws + o); };
  a.fl = f(w.fl); a.vlm = p.vl ? f(w.vlm) : nullptr; a.loc = f(w.loc); a.summ = f(w.summ); a.sfl = f(w.sfl);
  a.car = f(w.car);
  const bool mm_ro = s->readout == EWS_READOUT_MEAN || s->readout == EWS_READOUT_MAX;
  a.rows = bwd ? f(w.rows) : nullptr;
  a.rpart = mm_ro ? f(w.rpart) : nullptr;
  a.ridx = s->readout == EWS_READOUT_MAX ? (int*)(ws + w.ridx) : nullptr;
  a.amax = s->readout == EWS_READOUT_MAX ? (int*)(ws + w.amax) : nullptr;
  a.apow = f(w.apow);
  a.mflag = p.mats_int ? (int*)(ws + w.mflag) : nullptr;
  a.sflag = p.mats_smp ? (int*)(ws + w.sflag) : nullptr;
  a.ubuf = p.vl_int ? f(w.ubuf) : nullptr;
  if (bwd) {
    a.mu = f(w.mu); a.lend = f(w.lend); a.dloc = f(w.dloc);
    a.dfl = p.fl_int ? f(w.dfl) : nullptr; a.cpart = f(w.cpart); a.dvlm = p.vl_int ? f(w.dvlm) : nullptr;
    a.apart = f(w.apart); a.dv = f(w.dv); a.dhl = f(w.dhl); a.dhm = f(w.dhm); a.dsh = f(w.dsh);
    a.hpart = f(w.hpart); a.hsum = (double*)(ws + w.hsum);
    a.ebuf = p.vl_int ? f(w.ebuf) : nullptr;
  }
  return a;
}

#define WIDE_CHECK()                                            \
  do {                                                          \
    if (hipGetLastError() != hipSuccess) return EWS_ERR_LAUNCH; \
  } while (0)

int set_lds(const void* fn, size_t bytes) {
  return hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes) == hipSuccess
             ? EWS_OK : EWS_ERR_LAUNCH;
}

// forward passes: step matrices, local terms, chunk summaries, carries, rows (and the readout)
int run_forward(const WPlan& p, const WArgs& a, hipStream_t st) {
  const size_t lds = MF_ENT_FWD * sizeof(double);
  if (set_lds(reinterpret_cast<const void*>(&k_wmat), lds) != EWS_OK) return EWS_ERR_LAUNCH;
  // the powers table, the series path, then the matrices outside its radius (LDS forms)
  hipLaunchKernelGGL(k_wpowers, dim3(p.vl_int ? 2 : 1), dim3(NT), 0, st, a);
  if (p.mats_int) {
    hipLaunchKernelGGL(k_wmat_series, dim3((unsigned)std::min<long>((long)p.B * p.n, 1024)), dim3(NT), 0, st, a);
    hipLaunchKernelGGL(k_wmat, dim3((unsigned)p.g_int, p.gy_int), dim3(NT), lds, st, a, 2);
    WIDE_CHECK();
  }
  if (p.mats_smp) {
    hipLaunchKernelGGL(k_wmat_series_smp, dim3(p.B), dim3(NT), 0, st, a);
    hipLaunchKernelGGL(k_wmat, dim3(p.B, p.gy_smp), dim3(NT), lds, st, a, 0);
    WIDE_CHECK();
  }
  const dim3 gl((unsigned)std::min<long>((long)p.B * p.n, 4096)), gc(p.C, p.B);
  const size_t lds_leaf = (size_t)(lf_floats(p.rows, 2) + (p.vl_int ? LF_EXTRA : 0)) * 4;
  const void* kl = p.N == 1 ? (p.vl_int ? reinterpret_cast<const void*>(&k_wleaf<1, true>)
                                          : reinterpret_cast<const void*>(&k_wleaf<1, false>))
                            : (p.vl_int ? reinterpret_cast<const void*>(&k_wleaf<2, true>)
                                        : reinterpret_cast<const void*>(&k_wleaf<2, false>));
  if (set_lds(kl, lds_leaf) != EWS_OK) return EWS_ERR_LAUNCH;
  const dim3 gs(p.NSL, p.B);
  const size_t lds_vls = (size_t)VF_FLOATS * 4;
  if (p.N == 1) {
    if (p.vls) hipLaunchKernelGGL(k_wleaf_vls<1>, gs, dim3(NT), lds_vls, st, a);
    else if (p.vl_int) hipLaunchKernelGGL((k_wleaf<1, true>), gl, dim3(NT), lds_leaf, st, a);
    else hipLaunchKernelGGL((k_wleaf<1, false>), gl, dim3(NT), lds_leaf, st, a);
    hipLaunchKernelGGL((k_wscan<1, SCAN_SUMMARY>), gc, dim3(NT), 0, st, a);
    hipLaunchKernelGGL(k_wcarry<1>, dim3(p.B), dim3(NT), 0, st, a);
    hipLaunchKernelGGL((k_wscan<1, SCAN_ROWS>), gc, dim3(NT), 0, st, a);
  } else {
    if (p.vls) hipLaunchKernelGGL(k_wleaf_vls<2>, gs, dim3(NT), lds_vls, st, a);
    else if (p.vl_int) hipLaunchKernelGGL((k_wleaf<2, true>), gl, dim3(NT), lds_leaf, st, a);
    else hipLaunchKernelGGL((k_wleaf<2, false>), gl, dim3(NT), lds_leaf, st, a);
    hipLaunchKernelGGL((k_wscan<2, SCAN_SUMMARY>), gc, dim3(NT), 0, st, a);
    hipLaunchKernelGGL(k_wcarry<2>, dim3(p.B), dim3(NT), 0, st, a);
    hipLaunchKernelGGL((k_wscan<2, SCAN_ROWS>), gc, dim3(NT), 0, st, a);
  }
  WIDE_CHECK();
  if (a.readout == EWS_READOUT_TERMINAL || a.readout == EWS_READOUT_MEAN || a.readout == EWS_READOUT_MAX) {
    hipLaunchKernelGGL(k_wreadout, dim3((p.W + RO_COLS - 1) / RO_COLS, p.B), dim3(NT), 0, st, a);
    WIDE_CHECK();
  }
  return EWS_OK;
}

}  // namespace

bool eligible(const ews_dense_desc* s) {
  return s && s->dim > 16 && s->dim <= DP && s->depth >= 1 && s->depth <= 2 &&
         (s->leaf == EWS_LEAF_SERIES || s->leaf == EWS_LEAF_VAN_LOAN);
}

size_t workspace_bytes(const ews_dense_desc* s, bool backward) {
  WPlan p;
  if (plan(s, p) != EWS_OK) return 0;
  return layout(s, p, backward).total;
}

int forward(const ews_dense_desc* s, const float* path, const float* clock, const float* A, float* out,
            void* workspace, bool backward_layout, hipStream_t st) {
  WPlan p;
  const int rc = plan(s, p);
  if (rc != EWS_OK) return rc;
  if (!path || !clock || !A || !out || !workspace) return EWS_ERR_NULL;
  WArgs a = make_args(s, p, path, clock, A, out, workspace, backward_layout);
  return run_forward(p, a, st);
}

int backward(const ews_dense_desc* s, const float* path, const float* clock, const float* A, const float* grad_out,
             float* grad_path, float* grad_clock, float* grad_A, void* workspace, bool kept, hipStream_t st) {
  WPlan p;
  const int rc = plan(s, p);
  if (rc != EWS_OK) return rc;
  if (!path || !clock || !A || !grad_out || !grad_path || !grad_A || !workspace) return EWS_ERR_NULL;
  const WLay w = layout(s, p, true);
  WArgs a = make_args(s, p, path, clock, A, nullptr, workspace, true);
  a.gout = grad_out;
  if (!kept) {  // the forward again, with the padded prefix states kept (and the rows of the maxima of the max readout)
    WArgs f = a;
    if (s->readout == EWS_READOUT_MAX) f.out = (float*)((char*)workspace + w.outs);
    else f.readout = -1;  // no output: the states go to the workspace only
    const int r = run_forward(p, f, st);
    if (r != EWS_OK) return r;
  }
  const dim3 gc(p.C, p.B);
  const size_t lds_lb = (size_t)(lf_floats(p.rows, 4) + (p.vl_int ? LF_EXTRA : 0)) * 4;
  const int lk = !p.vl ? LK_SERIES : p.vl_int ? LK_VL_INT : LK_VL_SHARED;
  const void* kbs[2][3] = {{reinterpret_cast<const void*>(&k_wleaf_bwd<1, LK_SERIES>),
                            reinterpret_cast<const void*>(&k_wleaf_bwd<1, LK_VL_SHARED>),
                            reinterpret_cast<const void*>(&k_wleaf_bwd<1, LK_VL_INT>)},
                           {reinterpret_cast<const void*>(&k_wleaf_bwd<2, LK_SERIES>),
                            reinterpret_cast<const void*>(&k_wleaf_bwd<2, LK_VL_SHARED>),
                            reinterpret_cast<const void*>(&k_wleaf_bwd<2, LK_VL_INT>)}};
  if (set_lds(kbs[p.N - 1][lk], lds_lb) != EWS_OK) return EWS_ERR_LAUNCH;
  if (p.N == 1) {
    hipLaunchKernelGGL((k_wadj<1, ADJ_LOCAL>), gc, dim3(NT), 0, st, a);
    hipLaunchKernelGGL(k_wadj_carry<1>, dim3(p.B), dim3(NT), 0, st, a);
    hipLaunchKernelGGL((k_wadj<1, ADJ_FULL>), gc, dim3(NT), 0, st, a);
    if (p.vls) hipLaunchKernelGGL(k_wleaf_bwd_vls<1>, dim3(p.NSL, p.B), dim3(NT), (size_t)VB_FLOATS * 4, st, a);
    else if (lk == LK_SERIES)
      hipLaunchKernelGGL((k_wleaf_bwd<1, LK_SERIES>), dim3(p.NSL, p.B), dim3(NT), lds_lb, st, a);
    else if (lk == LK_VL_SHARED)
      hipLaunchKernelGGL((k_wleaf_bwd<1, LK_VL_SHARED>), dim3(p.NSL, p.B), dim3(NT), lds_lb, st, a);
    else hipLaunchKernelGGL((k_wleaf_bwd<1, LK_VL_INT>), dim3(p.NSL, p.B), dim3(NT), lds_lb, st, a);
  } else {
    hipLaunchKernelGGL((k_wadj<2, ADJ_LOCAL>), gc, dim3(NT), 0, st, a);
    hipLaunchKernelGGL(k_wadj_carry<2>, dim3(p.B), dim3(NT), 0, st, a);
    hipLaunchKernelGGL((k_wadj<2, ADJ_FULL>), gc, dim3(NT), 0, st, a);
    if (p.vls) hipLaunchKernelGGL(k_wleaf_bwd_vls<2>, dim3(p.NSL, p.B), dim3(NT), (size_t)VB_FLOATS * 4, st, a);
    else if (lk == LK_SERIES)
      hipLaunchKernelGGL((k_wleaf_bwd<2, LK_SERIES>), dim3(p.NSL, p.B), dim3(NT), lds_lb, st, a);
    else if (lk == LK_VL_SHARED)
      hipLaunchKernelGGL((k_wleaf_bwd<2, LK_VL_SHARED>), dim3(p.NSL, p.B), dim3(NT), lds_lb, st, a);
    else hipLaunchKernelGGL((k_wleaf_bwd<2, LK_VL_INT>), dim3(p.NSL, p.B), dim3(NT), lds_lb, st, a);
  }
  WIDE_CHECK();
  const long base = (long)p.B * p.NSL;
  if (set_lds(reinterpret_cast<const void*>(&k_wmat_bwd), MF_ENT_BWD_EXACT * 4) != EWS_OK) return EWS_ERR_LAUNCH;
  if (p.mats_int) {
    const size_t lds = (p.exact_int ? MF_ENT_BWD_EXACT : MF_ENT_BWD) * 4;
    hipLaunchKernelGGL(k_wmat_bwd_series, dim3((unsigned)p.g_ser), dim3(NT), 0, st, a);
    hipLaunchKernelGGL(k_wmat_bwd, dim3((unsigned)p.g_int, p.gy_int), dim3(NT), lds, st, a, 2, base);
    WIDE_CHECK();
  }
  if (p.mats_smp) {
    const size_t lds = (p.exact_smp ? MF_ENT_BWD_EXACT : MF_ENT_BWD) * 4;
    hipLaunchKernelGGL(k_wmat_bwd_series_smp, dim3(p.B), dim3(NT), 0, st, a, (int)p.g_ser);
    hipLaunchKernelGGL(k_wmat_bwd, dim3((unsigned)p.g_smp, p.gy_smp), dim3(NT), lds, st, a, 0,
                       base + p.g_int * p.gy_int);
    WIDE_CHECK();
  }
  // the series path's H_k: the per-interval workgroups' partials, then one per sample; one contraction into dA
  hipLaunchKernelGGL(k_whsum, dim3(PW + 1, MM / 64), dim3(NT), 0, st, a, (int)(p.g_ser + (p.mats_smp ? p.B : 0)));
  hipLaunchKernelGGL(k_wseries_dA, dim3(1), dim3(NT), 0, st, a, base + p.g_int * p.gy_int + p.g_smp * p.gy_smp);
  hipLaunchKernelGGL(k_wfinal_A, dim3(MM / 16), dim3(NT), 0, st, a, p.vl ? base : 0L,
                     base + p.g_int * p.gy_int + p.g_smp * p.gy_smp + 1, grad_A);
  hipLaunchKernelGGL(k_wknots, dim3((p.L + NT - 1) / NT, p.B), dim3(NT), 0, st, a, grad_path, grad_clock);
  WIDE_CHECK();
  return EWS_OK;
}

}  // namespace wide
}  // namespace ews
