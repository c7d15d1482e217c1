// Dense-generator EWS on MI355X (gfx950): any d x d generator A (d <= 16), depths 1-3, the series leaf.
//
// Reference path (sign convention of the reference: the flow over a clock step h is M = exp(-h A)):
//   local terms  ews/core/series_leaf.py:72-126 (letters b_0 = v, b_p = (-h/p) A b_{p-1};
//                level k = sum_{|m|<=q} c_m b_{m1} (x) ... (x) b_{mk}, c_m = prod_j 1/(M_j + k - j + 1))
//   flows        ews/core/chen_scan.py:155-168 (one exponential per interval, or one shared exponential)
//   Chen combine ews/core/chen_scan.py:125-214, ews/core/kernels/pallas_combine.py:603-749 (dense kernel)
//
// Passes (every array is padded to 16 channels; zero channels stay exactly zero through every step):
//   0  k_powers: table P_p = A^p / p! (float64 products, stored float32) and ||A||_1.
//      k_local: per interval (fully parallel) the levels s_1..s_N of the series leaf and the flow M_t.
//      Levels are built from nested degree sums instead of the coefficient tensor:
//         g1_n = b_n / (n+1),     g2_N = 1/(N+2) sum_{p+n=N} b_p (x) g1_n,
//         s_k  = sum_n bt^(k)_n (x) g_{k-1,n},   bt^(k)_n = sum_{p <= q-n} b_p / (p + n + k),
//      which is the same truncated sum (|m| <= q) as the reference's coefficient tensor.
//      Flows: Taylor polynomial of degree 12 in X = -h A / 2^s (||X||_1 <= 1), then s squarings.
//   1  k_scan<SUMMARY>: one workgroup per (sample, chunk) scans the chunk from a zero state; writes the chunk
//      summary and the chunk's flow product.
//   2  k_scan<PREFIX> over the chunk summaries (one chunk per sample): the carries (state before each chunk).
//   3  k_scan<PREFIX> from the carries: output rows (prefix), or the terminal row / mean / max.
//
// The Chen step in Horner form (level 3; the others are the same with fewer terms):
//     S3' = ((S3 x_3 M + S2 (x) s1) x_2 M + S1 (x) s2) x_1 M + s3
//     S2' = (S2 x_2 M + S1 (x) s1) x_1 M + s2,      S1' = M S1 + s1
// where x_a M applies M along tensor axis a: S2' = M S2 M^T + (M S1) s1^T + s2 and
// S3' = M^{(x)3} S3 + (M^{(x)2} S2) (x) s1 + (M S1) (x) s2 + s3, as in chen_scan.py:98-152.
// Mode products are 16x16x4 float32 MFMAs. The MFMA result registers of one mode product feed the next one
// directly: result lane l holds rows 4(l/16)+r (r = 0..3) of column l%16, and register r can be the B
// operand of k-step r with contraction index 4(l/16)+r (or the A operand, transposed), so only the axis-1
// product goes through LDS.
#include <hip/hip_runtime.h>

#include "ews_hip.h"
#include "ews_lanes.h"
#include "ews_wide.h"

namespace ews {
namespace dense {

constexpr int QMAX = 40;   // largest series order
constexpr int PM = 12;     // Taylor degree of the flow exponential (||X||_1 <= 1: error below 1/13! ~ 1.6e-10)
constexpr int SQMAX = 20;  // squarings of a scaled exponential at most (|h| ||A||_1 <= 2^20)
constexpr int RP = 20;     // LDS row pitch of the 16 x 16 slices (bank-conflict-free MFMA operand traffic)
constexpr int SP = 16 * RP + 4;  // LDS slice pitch of the level-3 buffers

__host__ __device__ constexpr int lw_of(int N) { return N == 1 ? 16 : (N == 2 ? 272 : 4368); }
#define LWN(N) lw_of(N)

typedef float f4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ f4 mfma(float a, float b, f4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}
// n floats from global memory into LDS by nt threads, eight loads in flight per thread before their stores (a
// loop of load-then-store waits out one memory latency per element)
__device__ __forceinline__ void stage_lds(float* dst, const float* src, int n, int tid, int nt) {
  for (int e0 = tid; e0 < n; e0 += 8 * nt) {
    float v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int e = e0 + u * nt;
      v[u] = e < n ? src[e] : 0.0f;
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int e = e0 + u * nt;
      if (e < n) dst[e] = v[u];
    }
  }
}
// LDS operations of one wavefront execute in program order: a compiler barrier orders a write before another
// lane's read of it
__device__ __forceinline__ void wave_order_d() { __builtin_amdgcn_wave_barrier(); }

struct Args {
  int B, L, n_int, d, N, q, flow_mode, readout, lvl0, W, LW;
  int T, C, npow;
  int leaf, vm, vl_expm, vl_mode, chen_expm;  // leaf kind; Van Loan knots M, its scheme and reweighting; flows' scheme
  const float* path;
  const float* clock;
  const float* A;
  float* apow;  // (npow, 256) P_p = A^p / p!, then one float ||A||_1
  float* loc;   // (B, n_int, LW) padded levels
  float* fl;    // (B, n_int, 256) flows
  float* summ;  // (B, C, LW)
  float* sfl;   // (B, C, 256)
  float* car;   // (B, C + 1, LW) state before chunk c (row C: terminal state)
  float* pre;   // (B, n_int, W) prefix rows (mean / max readouts)
  float* mats;  // (B, 3, 256) per-sample Van Loan step matrices P, V and the shared flow (uniform modes)
  // blocked carry scan: block summaries (B, NBc, LW), their flow products (B, NBc, 256), block carries (B, NBc + 1, LW)
  float* bsumm;
  float* bsfl;
  float* bcar;
  float* out;
  // backward: the adjoint scan's per-chunk local cotangents (B, C, LW), carries (B, C + 1, LW), max argmax (B, LW)
  float* lloc;
  float* lam;
  float* bagg;  // blocked adjoint carry scan: block local aggregates (B, NBc, LW), block-end cotangents (B, NBc + 1, LW)
  float* bl;
  int* amax;
  float* vlsave;  // backward's recompute: per interval the Van Loan P, V and knot increments (null otherwise)
};

// One scan over rows of (levels, flows): chunks of T rows, per-sample strides in floats.
struct Seq {
  const float* lv;
  long lv_bs;
  const float* fl;
  long fl_bs;
  int n, T;
  const float* init;  // per-chunk initial state: init + b * init_bs + c * LW (null: zero state)
  long init_bs;
  // PREFIX outputs: row t of sample b at rows + b * rows_bs + t * rows_ld (+ lvl0 leading 1.0 if set)
  float* rows;
  long rows_bs;
  int rows_ld, padded, lvl0, d;
  // SUMMARY outputs: (B, C, LW) states and (B, C, 256) flow products
  float* summ;
  float* sfl;
  int C;
};

// ------------------------------------------------------------------------------------------------ powers
// P_p = A^p / p! in float64 (stored float32), p < npow, zero-padded to 16 x 16; apow[npow * 256] = ||A||_1.
__global__ __launch_bounds__(256) void k_powers(Args a) {
  __shared__ double P[2][256];
  __shared__ double Ad[256];
  const int e = threadIdx.x, i = e >> 4, j = e & 15;
  Ad[e] = (i < a.d && j < a.d) ? (double)a.A[i * a.d + j] : 0.0;
  P[0][e] = (i == j) ? 1.0 : 0.0;
  a.apow[e] = (i == j) ? 1.0f : 0.0f;
  __syncthreads();
  for (int p = 1; p < a.npow; ++p) {
    const double* src = P[(p - 1) & 1];
    double acc = 0.0;
    for (int k = 0; k < 16; ++k) acc += src[i * 16 + k] * Ad[k * 16 + j];
    acc /= (double)p;
    P[p & 1][e] = acc;
    a.apow[p * 256 + e] = (float)acc;
    __syncthreads();
  }
  if (e < 16) {  // column sums, then max over columns (wave 0, lanes 0..15)
    double cs = 0.0;
    for (int r = 0; r < 16; ++r) cs += fabs(Ad[r * 16 + e]);
    for (int o = 8; o >= 1; o >>= 1) cs = fmax(cs, __shfl_xor(cs, o, 16));
    if (e == 0) a.apow[a.npow * 256] = (float)cs;
  }
}

// ------------------------------------------------------------------------------------------------ local terms
// Clock step of interval t of sample b for the flow: per interval, or the shared step of the cached modes
// (chen_scan.py:155-168); interval 0 of the basepoint mode has the identity flow (ident = true).
__device__ __forceinline__ float flow_step(const Args& a, const float* th, int t, bool& ident) {
  ident = false;
  if (a.flow_mode == EWS_FLOW_PER_INTERVAL) return th[t + 1] - th[t];
  if (a.flow_mode == EWS_FLOW_CACHED) return th[1] - th[0];
  ident = t == 0;
  return th[2] - th[1];
}

// One workgroup of 256 threads per interval (grid-stride loop). QB: compile-time bound on the series order
// (letters p <= q <= QB stay in registers / LDS with constant indices).
template <int N, int QB>
__global__ __launch_bounds__(256) void k_local(Args a) {
  __shared__ float sp[(QB > PM ? QB : PM) + 1][256];  // the powers table
  __shared__ float lt[QB + 1][16];   // letters b_p
  __shared__ float g1[QB + 1][16];   // b_n / (n + 1)
  __shared__ float bt[QB + 1][16];   // bt^(N)_n (the last level's left factors)
  __shared__ float vv[16];
  __shared__ float mm[256];
  const int tid = threadIdx.x, i = tid >> 4, j = tid & 15;
  const int q = a.q;
  stage_lds(&sp[0][0], a.apow, a.npow * 256, tid, 256);
  const float norm1 = a.apow[a.npow * 256];
  __syncthreads();
  const long total = (long)a.B * a.n_int;
  for (long it = blockIdx.x; it < total; it += gridDim.x) {
    const int b = (int)(it / a.n_int), t = (int)(it - (long)b * a.n_int);
    const float* th = a.clock + (size_t)b * a.L;
    const float h = th[t + 1] - th[t];
    if (tid < 16) {
      const float* x = a.path + ((size_t)b * a.L + t) * a.d;
      vv[tid] = tid < a.d ? x[a.d + tid] - x[tid] : 0.0f;
    }
    __syncthreads();
    // letters b_p = (-h)^p (P_p v)
    for (int e = tid; e < (q + 1) * 16; e += 256) {
      const int p = e >> 4, r = e & 15;
      float acc = 0.0f;
#pragma unroll
      for (int c = 0; c < 16; ++c) acc = fmaf(sp[p][r * 16 + c], vv[c], acc);
      float pw = 1.0f;
      for (int m = 0; m < p; ++m) pw *= -h;
      const float bp = acc * pw;
      lt[p][r] = bp;
      g1[p][r] = bp / (float)(p + 1);
    }
    __syncthreads();
    float* row = a.loc + ((size_t)b * a.n_int + t) * a.LW;
    if (tid < 16) {
      float s = 0.0f;
      for (int p = 0; p <= q; ++p) s += g1[p][tid];
      row[tid] = s;
    }
    if constexpr (N >= 2) {
      // bt_n = sum_{p <= q - n} b_p / (p + n + N); rows q < n <= QB are zero (read by the unrolled sums below)
      for (int e = tid; e < (QB + 1) * 16; e += 256) {
        const int n = e >> 4, r = e & 15;
        float s = 0.0f;
        for (int p = 0; p + n <= q; ++p) s += lt[p][r] / (float)(p + n + N);
        bt[n][r] = s;
      }
      __syncthreads();
      if constexpr (N == 2) {
        // s2[i][j] = sum_n bt_n[i] g1_n[j]
        float s = 0.0f;
        for (int n = 0; n <= q; ++n) s = fmaf(bt[n][i], g1[n][j], s);
        row[16 + tid] = s;
      } else {
        // g2_M[i][j] = 1/(M+2) sum_{p+n=M} b_p[i] g1_n[j]; s2 = sum_M g2_M; s3[c][i][j] = sum_M bt_M[c] g2_M[i][j]
        float G[QB + 1];
        float s2 = 0.0f;
#pragma unroll
        for (int M = 0; M <= QB; ++M) {
          float s = 0.0f;
          if (M <= q) {
#pragma unroll
            for (int p = 0; p <= M; ++p) s = fmaf(lt[p][i], g1[M - p][j], s);
            s /= (float)(M + 2);
          }
          G[M] = s;
          s2 += s;
        }
        row[16 + tid] = s2;
#pragma unroll 4
        for (int c = 0; c < 16; ++c) {
          float s = 0.0f;
#pragma unroll
          for (int M = 0; M <= QB; ++M) s = fmaf(bt[M][c], G[M], s);
          row[272 + c * 256 + tid] = s;
        }
      }
    }
    // flow M_t = exp(-h_f A): Taylor of degree PM in X = -h_f A / 2^s, then s squarings
    {
      bool ident;
      const float hf = flow_step(a, th, t, ident);
      float* fr = a.fl + ((size_t)b * a.n_int + t) * 256;
      if (ident) {
        fr[tid] = (i == j) ? 1.0f : 0.0f;
      } else {
        int s = 0;
        float x = fabsf(hf) * norm1;
        while (x > 1.0f && s < SQMAX) {
          x *= 0.5f;
          ++s;
        }
        const float y = -hf * ldexpf(1.0f, -s);
        float acc = sp[PM][tid];
#pragma unroll
        for (int p = PM - 1; p >= 0; --p) acc = fmaf(acc, y, sp[p][tid]);
        for (int r = 0; r < s; ++r) {
          __syncthreads();
          mm[tid] = acc;
          __syncthreads();
          float v = 0.0f;
#pragma unroll
          for (int c = 0; c < 16; ++c) v = fmaf(mm[i * 16 + c], mm[c * 16 + j], v);
          acc = v;
        }
        fr[tid] = acc;
      }
    }
    __syncthreads();
  }
}

// Depth-3 local terms on MFMA, one wavefront per interval (four per workgroup, grid-stride). The letters come
// from the recursion b_p = (-h/p) A b_{p-1} (lane (c16, g) holds A[c16][4g .. 4g+3]); the degree-N blocks
// g2_N = 1/(N+2) sum_{p <= N} b_p (x) g1_{N-p} are MFMAs with the contraction over p; four degree slices at a
// time go through LDS and feed the level-3 contraction s3[a][i][j] = sum_N bt_N[a] g2_N[i][j] (one k-step of
// four degrees per slice set, sixteen output tiles, tile i holding s3[.][i][.]). Rows p > q of the letter
// buffer stay zero, so the unrolled k-steps over whole groups of four degrees add nothing beyond the order q.
// Three workgroups per CU fit the LDS of the orders up to 24; the order-40 tables hold two.
template <int QB>
__global__ __launch_bounds__(256, QB <= 24 ? 3 : 2) void k_local3(Args a) {
  constexpr int QB4 = (QB + 4) / 4 * 4;  // letter rows 0 .. QB4-1 (QB + 1 rounded up to whole k-steps)
  constexpr int G2S = 16 * RP + 16;      // LDS floats per degree slice (row pitch RP; slices on offset banks)
  constexpr int NINV = 2 * QB4 + 8;      // reciprocals 1/n, n < NINV (no divisions in the loops)
  __shared__ __align__(16) float sp[PM + 1][256];   // P_p = A^p / p!, p <= PM (flows; P_1 = A)
  __shared__ __align__(16) float lt[4][QB4 * 16];   // letters b_p of each wave's interval
  __shared__ __align__(16) float gt[4][QB4 * 16];   // g1_n = b_n / (n + 1)
  __shared__ __align__(16) float g2b[4][4 * G2S];   // four degree slices of g2 per wave (then the flow squarings)
  __shared__ float inv[NINV];
  const int tid = threadIdx.x, w = tid >> 6, l = tid & 63, g = l >> 4, c16 = l & 15;
  const int q = a.q;
  stage_lds(&sp[0][0], a.apow, (PM + 1) * 256, tid, 256);
  for (int e = tid; e < NINV; e += 256) inv[e] = e ? 1.0f / (float)e : 0.0f;
  const float norm1 = a.apow[a.npow * 256];
  float* L = lt[w];
  float* G1 = gt[w];
  float* G2 = g2b[w];
  for (int e = l; e < QB4 * 16; e += 64) L[e] = G1[e] = 0.0f;
  __syncthreads();
  const f4 a4 = *reinterpret_cast<const f4*>(&sp[1][c16 * 16 + 4 * g]);  // A[c16][4g .. 4g+3]
  const long total = (long)a.B * a.n_int;
  // the interval's clock values and increment coordinates are loaded one interval ahead into registers, so that no
  // memory round trip sits at the top of an interval
  const long first = (long)blockIdx.x * 4 + w, stride = (long)gridDim.x * 4;
  float nth0 = 0.0f, nth1 = 0.0f, nx0 = 0.0f, nx1 = 0.0f;
  const bool xl = l < 16 && l < a.d;
  auto prefetch = [&](long i2) {
    const int b2 = (int)(i2 / a.n_int), t2 = (int)(i2 - (long)b2 * a.n_int);
    const float* th2 = a.clock + (size_t)b2 * a.L + t2;
    nth0 = th2[0];
    nth1 = th2[1];
    if (xl) {
      const float* x = a.path + ((size_t)b2 * a.L + t2) * a.d;
      nx0 = x[l];
      nx1 = x[a.d + l];
    }
  };
  if (first < total) prefetch(first);
  for (long it = first; it < total; it += stride) {
    const int b = (int)(it / a.n_int), t = (int)(it - (long)b * a.n_int);
    const float* th = a.clock + (size_t)b * a.L;
    const float h = nth1 - nth0;
    const float v = xl ? nx1 - nx0 : 0.0f;
    if (it + stride < total) prefetch(it + stride);
    wave_order_d();  // the previous interval's reads of L / G1 / G2 come first
    if (l < 16) {
      L[l] = v;
      G1[l] = v;
    }
    wave_order_d();
    for (int pp = 1; pp <= q; ++pp) {
      const f4 bp = *reinterpret_cast<const f4*>(L + (pp - 1) * 16 + 4 * g);
      float sm = fmaf(a4.x, bp.x, fmaf(a4.y, bp.y, fmaf(a4.z, bp.z, a4.w * bp.w)));
      sm = lanes::add_xor32(lanes::add_xor16(sm));
      const float bv = sm * (-h * inv[pp]);
      if (g == 0) L[pp * 16 + c16] = bv;
      if (g == 1) G1[pp * 16 + c16] = bv * inv[pp + 1];
      wave_order_d();
    }
    float* row = a.loc + ((size_t)b * a.n_int + t) * a.LW;
    if (l < 16) {
      float sm = 0.0f;
      for (int n = 0; n <= q; ++n) sm += G1[n * 16 + l];
      row[l] = sm;
    }
    f4 acc3[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) acc3[i] = f4{0.0f, 0.0f, 0.0f, 0.0f};
    f4 s2acc = {0.0f, 0.0f, 0.0f, 0.0f};
    const int nks = (q + 4) / 4;  // k-steps that hold a degree <= q
#pragma unroll 1
    for (int ks = 0; ks < nks; ++ks) {
      // A operand of this level-3 k-step: bt_N[c16] = sum_{p <= q - N} b_p[c16] / (p + N + 3), N = 4 ks + g
      float btv = 0.0f;
      {
        const int N = 4 * ks + g;
        for (int pp = 0; pp + N <= q; ++pp) btv = fmaf(L[pp * 16 + c16], inv[pp + N + 3], btv);
      }
      // the four degrees N = 4 ks + nn as independent accumulators: one letter column b_p (p = 4 kp + g) per
      // k-step serves all four (g1_{N-p} is zero for p > N; degrees above q come out zero)
      f4 dd[4];
#pragma unroll
      for (int nn = 0; nn < 4; ++nn) dd[nn] = f4{0.0f, 0.0f, 0.0f, 0.0f};
      for (int kp = 0; kp <= ks; ++kp) {
        const int pp = 4 * kp + g;
        const float av = L[pp * 16 + c16];  // b_p[i]
#pragma unroll
        for (int nn = 0; nn < 4; ++nn) {
          const int n = 4 * ks + nn - pp;
          const float bv = (n >= 0 && 4 * ks + nn <= q) ? G1[max(n, 0) * 16 + c16] : 0.0f;  // g1_{N-p}[j]
          dd[nn] = mfma(av, bv, dd[nn]);
        }
      }
#pragma unroll
      for (int nn = 0; nn < 4; ++nn) {
        const float sc = inv[4 * ks + nn + 2];
#pragma unroll
        for (int r = 0; r < 4; ++r) dd[nn][r] *= sc;
        s2acc += dd[nn];
#pragma unroll
        for (int r = 0; r < 4; ++r) G2[nn * G2S + (4 * g + r) * RP + c16] = dd[nn][r];
      }
      wave_order_d();
      // tile i, transposed: rows j, columns a (A operand g2_N[i][j], B operand bt_N[a]), so that the lane's four
      // result registers are s3[c16][i][4g .. 4g+3], one 16-byte store
      const float* gs = G2 + g * G2S;
#pragma unroll
      for (int i = 0; i < 16; ++i) acc3[i] = mfma(gs[i * RP + c16], btv, acc3[i]);
      wave_order_d();
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) row[16 + (4 * g + r) * 16 + c16] = s2acc[r];
#pragma unroll
    for (int i = 0; i < 16; ++i) *reinterpret_cast<f4*>(row + 272 + c16 * 256 + i * 16 + 4 * g) = acc3[i];
    // flow M_t = exp(-h_f A): Taylor of degree PM in X = -h_f A / 2^s (lane: entries 4l .. 4l+3), s squarings
    {
      bool ident = false;
      const float hf = a.flow_mode == EWS_FLOW_PER_INTERVAL ? h : flow_step(a, th, t, ident);
      float* fr = a.fl + ((size_t)b * a.n_int + t) * 256;
      f4 m;
      if (ident) {
#pragma unroll
        for (int r = 0; r < 4; ++r) m[r] = ((4 * l + r) >> 4) == ((4 * l + r) & 15) ? 1.0f : 0.0f;
      } else {
        int sq = 0;
        float x = fabsf(hf) * norm1;
        while (x > 1.0f && sq < SQMAX) {
          x *= 0.5f;
          ++sq;
        }
        const float y = -hf * ldexpf(1.0f, -sq);
        m = *reinterpret_cast<const f4*>(&sp[PM][4 * l]);
#pragma unroll
        for (int pp = PM - 1; pp >= 0; --pp) {
          const f4 c = *reinterpret_cast<const f4*>(&sp[pp][4 * l]);
#pragma unroll
          for (int r = 0; r < 4; ++r) m[r] = fmaf(m[r], y, c[r]);
        }
        float* mm = g2b[w];  // the degree slices are done
        const int i = l >> 2, j0 = 4 * (l & 3);
        for (int r2 = 0; r2 < sq; ++r2) {
          *reinterpret_cast<f4*>(mm + 4 * l) = m;
          wave_order_d();
          f4 v = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
          for (int cc = 0; cc < 16; ++cc) {
            const float mic = mm[i * 16 + cc];
            const f4 mr = *reinterpret_cast<const f4*>(mm + cc * 16 + j0);
#pragma unroll
            for (int r = 0; r < 4; ++r) v[r] = fmaf(mic, mr[r], v[r]);
          }
          wave_order_d();
          m = v;
        }
      }
      *reinterpret_cast<f4*>(fr + 4 * l) = m;
    }
  }
}

// ------------------------------------------------------------------------------------------------ matrix functions
// Wavefront-level functions of the zero-padded 16 x 16 generator (powers table sp: P_p = A^p / p! in LDS, so
// sp[1] = A and sp[2] = A^2 / 2). Results are row-major 16 x 16 in per-wave LDS buffers; lane l owns entries
// 4l .. 4l+3 (row l/4, columns 4(l%4) ..) in the elementwise parts.
typedef float LdsTable[256];

// E = exp(-c A) and, when Phi is set, Phi = phi(-c A) = sum_p (-c A)^p / (p+1)!: Taylor polynomials of degree
// PM in X = -c A / 2^s (||X||_1 <= 1), then s doublings E <- E E, Phi <- (Phi + Phi E) / 2
// (phi(2X) = phi(X) (I + e^X) / 2).
__device__ __forceinline__ void wave_expm(const LdsTable* sp, float norm1, float c, float* E, float* Phi, int l) {
  int s = 0;
  float x = fabsf(c) * norm1;
  while (x > 1.0f && s < SQMAX) {
    x *= 0.5f;
    ++s;
  }
  const float y = -c * ldexpf(1.0f, -s);
  f4 e = *reinterpret_cast<const f4*>(&sp[PM][4 * l]);
  f4 f = e * (1.0f / (float)(PM + 1));
#pragma unroll
  for (int p = PM - 1; p >= 0; --p) {
    const f4 t = *reinterpret_cast<const f4*>(&sp[p][4 * l]);
    const float ip = 1.0f / (float)(p + 1);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      e[r] = fmaf(e[r], y, t[r]);
      f[r] = fmaf(f[r], y, t[r] * ip);
    }
  }
  const int i = l >> 2, j0 = 4 * (l & 3);
  for (int r2 = 0; r2 < s; ++r2) {
    *reinterpret_cast<f4*>(E + 4 * l) = e;
    if (Phi) *reinterpret_cast<f4*>(Phi + 4 * l) = f;
    wave_order_d();
    f4 ne = {0.0f, 0.0f, 0.0f, 0.0f}, nf = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      const f4 ek = *reinterpret_cast<const f4*>(E + k * 16 + j0);
      const float eik = E[i * 16 + k];
#pragma unroll
      for (int r = 0; r < 4; ++r) ne[r] = fmaf(eik, ek[r], ne[r]);
      if (Phi) {
        const float fik = Phi[i * 16 + k];
#pragma unroll
        for (int r = 0; r < 4; ++r) nf[r] = fmaf(fik, ek[r], nf[r]);
      }
    }
    wave_order_d();
    e = ne;
#pragma unroll
    for (int r = 0; r < 4; ++r) f[r] = 0.5f * (f[r] + nf[r]);
  }
  *reinterpret_cast<f4*>(E + 4 * l) = e;
  if (Phi) *reinterpret_cast<f4*>(Phi + 4 * l) = f;
  wave_order_d();
}

// out = (I + alpha A + beta A^2)^{-1} by Gauss-Jordan elimination on [N | I] with partial pivoting (largest
// magnitude in the column among the rows not yet used, ties to the lower row); rows are not swapped, the
// pivot order is undone when the result is written. Lane (r, g) holds row r, columns 8g .. 8g+7 of [N | I].
// xch: 8 floats x 4 groups of LDS for the pivot row.
__device__ __forceinline__ void wave_inverse(const LdsTable* sp, float alpha, float beta, float* out, float* xch, int l) {
  const int r = l & 15, g = l >> 4;
  float m[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int col = 8 * g + j;
    if (g < 2)
      m[j] = (r == col ? 1.0f : 0.0f) + alpha * sp[1][r * 16 + col] + 2.0f * beta * sp[2][r * 16 + col];
    else
      m[j] = (r == col - 16) ? 1.0f : 0.0f;
  }
  bool used = false;
  int krow = 0;
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    const float colv = __shfl(m[k & 7], r + 16 * (k >> 3), 64);  // N'[r][k]
    float cand = used ? -1.0f : fabsf(colv);
    int crow = r;
#pragma unroll
    for (int o = 1; o < 16; o <<= 1) {
      const float oc = __shfl_xor(cand, o, 64);
      const int orow = __shfl_xor(crow, o, 64);
      if (oc > cand || (oc == cand && orow < crow)) {
        cand = oc;
        crow = orow;
      }
    }
    const int p = __builtin_amdgcn_readfirstlane(crow);
    const float pv = __shfl(colv, p, 64);
    if (r == p) {
#pragma unroll
      for (int j = 0; j < 8; ++j) m[j] = m[j] / pv;
      used = true;
      krow = k;
      *reinterpret_cast<f4*>(xch + 8 * g) = f4{m[0], m[1], m[2], m[3]};
      *reinterpret_cast<f4*>(xch + 8 * g + 4) = f4{m[4], m[5], m[6], m[7]};
    }
    wave_order_d();
    const f4 lo = *reinterpret_cast<const f4*>(xch + 8 * g);
    const f4 hi = *reinterpret_cast<const f4*>(xch + 8 * g + 4);
    wave_order_d();
    if (r != p) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        m[j] = fmaf(-colv, lo[j], m[j]);
        m[j + 4] = fmaf(-colv, hi[j], m[j + 4]);
      }
    }
  }
  // the rows' right halves are the rows of the inverse in pivot order: row r holds inverse row krow
  if (g >= 2) {
    float* o = out + krow * 16 + 8 * (g - 2);
    *reinterpret_cast<f4*>(o) = f4{m[0], m[1], m[2], m[3]};
    *reinterpret_cast<f4*>(o + 4) = f4{m[4], m[5], m[6], m[7]};
  }
  wave_order_d();
}

// Power-series form of the matrix functions below: each is analytic in a = c A at 0, sum_k b_k a^k =
// sum_k (b_k c^k k!) P_k with the table P_k = A^k / k!, evaluated elementwise (no cross-lane traffic). Used when
// x = |c| ||A||_1 keeps the 13-term remainder below ~1e-8 relative: exact x <= 1 (x^13 e^x / 13!); cayley
// x <= 0.48 (poles of (1 + a/2)^{-1} at |a| = 2); euler x <= 0.24 (|a| = 1; the euler flow I - cA is a
// polynomial); pade x <= 0.7 (poles of (1 + a/2 + a^2/12)^{-1} at |a| = sqrt 12).
__device__ __forceinline__ bool series_fits(int scheme, float x, bool flow) {
  switch (scheme) {
    case EWS_EXPM_EXACT: return x <= 1.0f;
    case EWS_EXPM_EULER: return flow || x <= 0.24f;
    case EWS_EXPM_CAYLEY: return x <= 0.48f;
    default: return x <= 0.7f;
  }
}

// Coefficients b_k in a (then scaled by c^k k!), for P and V of wave_matfn:
//   exact   P: (-1)^k / k!             V: (-1)^k / (k+1)!
//   cayley  V: (-1/2)^k                P: 2V - I
//   euler   V = P: (-1)^k              flow: 1, -1
//   pade    V: b_0 = 1, b_1 = -1/2, b_k = -(b_{k-1}/2 + b_{k-2}/12)  (1 / (1 + a/2 + a^2/12))
//           P = I - a V: 1, -b_{k-1}
__device__ __forceinline__ void series_mats(const LdsTable* sp, int scheme, float c, bool flow, float* P, float* V,
                                            int l) {
  float cp[PM + 1], cv[PM + 1];
  float fact = 1.0f, sgn = 1.0f, half = 1.0f, b1 = 0.0f, b2 = 0.0f;
#pragma unroll
  for (int k = 0; k <= PM; ++k) {
    if (k) {
      fact *= (float)k;
      sgn = -sgn;
      half *= -0.5f;
    }
    float bp, bv;
    if (scheme == EWS_EXPM_EXACT) {
      bv = sgn / (fact * (float)(k + 1));
      bp = sgn / fact;
    } else if (scheme == EWS_EXPM_CAYLEY) {
      bv = half;
      bp = k ? 2.0f * half : 1.0f;
    } else if (scheme == EWS_EXPM_EULER) {
      bv = sgn;
      bp = flow ? (k == 0 ? 1.0f : (k == 1 ? -1.0f : 0.0f)) : sgn;
    } else {
      bv = k == 0 ? 1.0f : (k == 1 ? -0.5f : -(0.5f * b1 + b2 * (1.0f / 12.0f)));
      bp = k == 0 ? 1.0f : -b1;
      b2 = b1;
      b1 = bv;
    }
    cp[k] = bp;
    cv[k] = bv;
  }
  float sc = 1.0f;
#pragma unroll
  for (int k = 1; k <= PM; ++k) {
    sc *= c * (float)k;
    cp[k] *= sc;
    cv[k] *= sc;
  }
  f4 ap = {0.0f, 0.0f, 0.0f, 0.0f}, av = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int k = PM; k >= 0; --k) {  // smallest terms first
    const f4 t = *reinterpret_cast<const f4*>(&sp[k][4 * l]);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      ap[r] = fmaf(cp[k], t[r], ap[r]);
      av[r] = fmaf(cv[k], t[r], av[r]);
    }
  }
  *reinterpret_cast<f4*>(P + 4 * l) = ap;
  if (!flow) *reinterpret_cast<f4*>(V + 4 * l) = av;
  wave_order_d();
}

// Just outside a rational scheme's series radius (x = |c| ||A||_1 below 0.85 of it) the truncated series of
// N^{-1} still has a residual E = I - N X below 1/2, and Newton-Schulz iterations X <- X (2I - N X) square it
// (I - N X' = E^2): a few 16 x 16 products instead of a Gauss-Jordan elimination. iters: the squarings that take the
// bound ||E|| <= x_r^13 / (1 - x_r) (1 + x), x_r = x / radius, below 1e-9.
__device__ __forceinline__ bool ns_iters(int scheme, float x, int& iters) {
  const float rho = scheme == EWS_EXPM_CAYLEY ? 2.0f : (scheme == EWS_EXPM_EULER ? 1.0f : 3.4641016f);
  const float r = x / rho;
  if (!(r < 0.85f)) return false;
  float r13 = r;
#pragma unroll
  for (int k = 1; k < 13; ++k) r13 *= r;
  float e = r13 / (1.0f - r) * (1.0f + x);
  if (!(e < 0.5f)) return false;
  iters = 0;
  while (e > 1e-9f && iters < 6) {
    e *= e;
    ++iters;
  }
  return true;
}

// X <- X (2I - N X), iters times, N = I + alpha A + beta A^2 (from the table: A = P_1, A^2 = 2 P_2); X in LDS
// (row-major 16 x 16), R: 256 floats of LDS scratch.
__device__ __forceinline__ void wave_ns(const LdsTable* sp, float alpha, float beta, float* X, float* R, int iters,
                                        int l) {
  const int i = l >> 2, j0 = 4 * (l & 3);
  for (int it = 0; it < iters; ++it) {
    f4 y = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      const float nik = (i == k ? 1.0f : 0.0f) + alpha * sp[1][i * 16 + k] + 2.0f * beta * sp[2][i * 16 + k];
      const f4 xk = *reinterpret_cast<const f4*>(X + k * 16 + j0);
#pragma unroll
      for (int r = 0; r < 4; ++r) y[r] = fmaf(nik, xk[r], y[r]);
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) y[r] = (i == j0 + r ? 2.0f : 0.0f) - y[r];
    *reinterpret_cast<f4*>(R + 4 * l) = y;
    wave_order_d();
    f4 z = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      const float xik = X[i * 16 + k];
      const f4 rk = *reinterpret_cast<const f4*>(R + k * 16 + j0);
#pragma unroll
      for (int r = 0; r < 4; ++r) z[r] = fmaf(xik, rk[r], z[r]);
    }
    wave_order_d();
    *reinterpret_cast<f4*>(X + 4 * l) = z;
    wave_order_d();
  }
}

// The matrix functions of one step c under a scheme of ews/core/expm_approx.py:13-41.
//   flow = true:  P = expm_scheme(-c A):   exact exp(-cA); euler I - cA; cayley (I + cA/2)^{-1} (I - cA/2)
//                 = 2 (I + cA/2)^{-1} - I; pade (I + cA/2 + c^2A^2/12)^{-1} (I - cA/2 + c^2A^2/12)
//                 = I - c (I + cA/2 + c^2A^2/12)^{-1} A.
//   flow = false: the Van Loan step of van_loan.py:31-71 with a = c A (c = dt / M): the augmented exponential
//                 E = expm_scheme([[a, w], [0, 0]]) = [[C, u], [0, 1]]; the knot increments are
//                 Delta_m = C^{m-1-M} u (m = 1..M), so Delta_M = C^{-1} u = V w and Delta_{m-1} = P Delta_m with
//                 P = C^{-1}:
//                   exact  P = exp(-a), V = phi(-a);        cayley V = (I + a/2)^{-1}, P = 2V - I;
//                   euler  V = (I + a)^{-1}, P = V;         pade   V = (I + a/2 + a^2/12)^{-1}, P = I - V a.
// Buffers: P and V (V only for flow = false) 256 floats, T 256 + 32 floats of scratch.
__device__ __forceinline__ void wave_matfn(const LdsTable* sp, float norm1, int scheme, float c, bool flow, float* P, float* V,
                           float* T, int l) {
  if (series_fits(scheme, fabsf(c) * norm1, flow)) {
    series_mats(sp, scheme, c, flow, P, V, l);
    return;
  }
  if (scheme == EWS_EXPM_EXACT) {
    wave_expm(sp, norm1, c, P, flow ? nullptr : V, l);
    return;
  }
  const int i = l >> 2, j0 = 4 * (l & 3);
  if (scheme == EWS_EXPM_EULER && flow) {
    f4 e;
#pragma unroll
    for (int r = 0; r < 4; ++r) e[r] = (i == j0 + r ? 1.0f : 0.0f) - c * sp[1][4 * l + r];
    *reinterpret_cast<f4*>(P + 4 * l) = e;
    wave_order_d();
    return;
  }
  const float alpha = scheme == EWS_EXPM_EULER ? c : 0.5f * c;
  const float beta = scheme == EWS_EXPM_PADE ? c * c * (1.0f / 12.0f) : 0.0f;
  float* inv = flow ? T : V;
  int nsit;
  if (ns_iters(scheme, fabsf(c) * norm1, nsit)) {
    series_mats(sp, scheme, c, false, P, inv, l);  // the truncated series of N^{-1} (P is scratch here)
    wave_ns(sp, alpha, beta, inv, P, nsit, l);
  } else {
    wave_inverse(sp, alpha, beta, inv, T + 256, l);
  }
  const f4 vi = *reinterpret_cast<const f4*>(inv + 4 * l);
  f4 e;
  if (scheme == EWS_EXPM_CAYLEY) {
#pragma unroll
    for (int r = 0; r < 4; ++r) e[r] = 2.0f * vi[r] - (i == j0 + r ? 1.0f : 0.0f);
  } else if (scheme == EWS_EXPM_EULER) {
    e = vi;
  } else {  // pade: I - c inv A
    f4 va = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      const float ik = inv[i * 16 + k];
      const f4 ak = *reinterpret_cast<const f4*>(&sp[1][k * 16 + j0]);
#pragma unroll
      for (int r = 0; r < 4; ++r) va[r] = fmaf(ik, ak[r], va[r]);
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) e[r] = (i == j0 + r ? 1.0f : 0.0f) - c * va[r];
  }
  wave_order_d();
  *reinterpret_cast<f4*>(P + 4 * l) = e;
  wave_order_d();
}

__device__ __forceinline__ void wave_identity(float* P, int l) {
  f4 e;
#pragma unroll
  for (int r = 0; r < 4; ++r) e[r] = ((4 * l + r) >> 4) == ((4 * l + r) & 15) ? 1.0f : 0.0f;
  *reinterpret_cast<f4*>(P + 4 * l) = e;
  wave_order_d();
}

// Van Loan step of the uniform reweightings (van_loan.py:91-160): dt = interval_times[0] (uniform) or
// interval_times[1] (uniform_basepoint, whose interval 0 is the pure jump); a step dt <= 1e-12 is the jump
// (linear knots, P = V = I).
__device__ __forceinline__ float vl_shared_step(const Args& a, const float* th) {
  const float dt = a.vl_mode == EWS_FLOW_CACHED ? th[1] - th[0] : th[2] - th[1];
  return dt > 1e-12f ? dt / (float)a.vm : 0.0f;
}

// Per-sample matrices of the uniform modes, one wavefront per sample: the Van Loan P and V of the shared step
// (mats[b][0], mats[b][1]) and the shared flow (mats[b][2]) of the cached flow modes.
__global__ __launch_bounds__(64) void k_prep(Args a) {
  __shared__ __align__(16) float sp[PM + 1][256];
  __shared__ __align__(16) float P[256], V[256], T[256 + 32];
  const int l = threadIdx.x, b = blockIdx.x;
  stage_lds(&sp[0][0], a.apow, (PM + 1) * 256, l, 64);
  const float norm1 = a.apow[a.npow * 256];
  __syncthreads();
  const float* th = a.clock + (size_t)b * a.L;
  float* mb = a.mats + (size_t)b * 768;
  if (a.leaf == EWS_LEAF_VAN_LOAN && a.vl_mode != EWS_FLOW_PER_INTERVAL) {
    wave_matfn(sp, norm1, a.vl_expm, vl_shared_step(a, th), false, P, V, T, l);
    *reinterpret_cast<f4*>(mb + 4 * l) = *reinterpret_cast<const f4*>(P + 4 * l);
    *reinterpret_cast<f4*>(mb + 256 + 4 * l) = *reinterpret_cast<const f4*>(V + 4 * l);
    wave_order_d();
  }
  if (a.flow_mode != EWS_FLOW_PER_INTERVAL) {
    bool ident;
    const float hf = flow_step(a, th, 1, ident);
    wave_matfn(sp, norm1, a.chen_expm, hf, true, P, nullptr, T, l);
    *reinterpret_cast<f4*>(mb + 512 + 4 * l) = *reinterpret_cast<const f4*>(P + 4 * l);
  }
}

// Flow M_t = expm_scheme(-h_t A) of interval t under chen_expm (chen_scan.py:155-168), written to its row of fl
// by one wavefront: computed per interval, the per-sample copy of the cached modes, or the identity of interval 0
// of the basepoint mode. P (256) and T (256 + 32) are the wave's LDS scratch.
__device__ __forceinline__ void write_flow(const Args& a, const LdsTable* sp, float norm1, int b, int t,
                                           const float* th, float* P, float* T, int l) {
  bool ident;
  const float hf = flow_step(a, th, t, ident);
  f4 m;
  if (ident) {
#pragma unroll
    for (int r = 0; r < 4; ++r) m[r] = ((4 * l + r) >> 4) == ((4 * l + r) & 15) ? 1.0f : 0.0f;
  } else if (a.flow_mode != EWS_FLOW_PER_INTERVAL) {
    m = *reinterpret_cast<const f4*>(a.mats + (size_t)b * 768 + 512 + 4 * l);
  } else {
    wave_matfn(sp, norm1, a.chen_expm, hf, true, P, nullptr, T, l);
    m = *reinterpret_cast<const f4*>(P + 4 * l);
    wave_order_d();
  }
  *reinterpret_cast<f4*>(a.fl + ((size_t)b * a.n_int + t) * 256 + 4 * l) = m;
}

// Flows of a scheme other than the series kernels' fused exact ones, one wavefront per interval.
__global__ __launch_bounds__(256) void k_flows(Args a) {
  __shared__ __align__(16) float sp[PM + 1][256];
  __shared__ __align__(16) float Pw[4][256], Tw[4][256 + 32];
  const int tid = threadIdx.x, w = tid >> 6, l = tid & 63;
  stage_lds(&sp[0][0], a.apow, (PM + 1) * 256, tid, 256);
  const float norm1 = a.apow[a.npow * 256];
  __syncthreads();
  const long total = (long)a.B * a.n_int;
  for (long it = (long)blockIdx.x * 4 + w; it < total; it += (long)gridDim.x * 4) {
    const int b = (int)(it / a.n_int), t = (int)(it - (long)b * a.n_int);
    write_flow(a, sp, norm1, b, t, a.clock + (size_t)b * a.L, Pw[w], Tw[w], l);
  }
}

// ------------------------------------------------------------------------------------------------ Van Loan leaf
// One wavefront per interval (grid-stride). The knot increments Delta_1..Delta_M of the reweighted path
// (van_loan.py:31-160: knots K_m = W E^m[:d, d], W = (E^M[:d, :d])^{-1}) are Delta_M = V w, Delta_{m-1} = P Delta_m
// with w = v / M (see wave_matfn), and the levels are the signature of the piecewise-linear path through the
// knots (signature.py:20-35): the Chen product of the segments' exponentials, which in closed form is
//   S1 = sum_m Delta_m,   S2 = sum_m Y_m (x) Delta_m,
//   S3 = sum_m (Y_m (x) Delta_m (x) R_m + X_m (x) Delta_m (x) Delta_m / 2)
// with the exclusive prefix sums Pre_m = sum_{j<m} Delta_j (= S1 - R_m - Delta_m), suffix sums
// R_m = sum_{j>m} Delta_j, Y_m = Pre_m + Delta_m / 2 and X_m = Pre_m + Delta_m / 3 (segment m contributes
// Delta^{(x)2}/2 and Delta^{(x)3}/6 and meets the segments before and after it). S2 and S3 are 16x16x4 float32
// MFMAs contracting over the segment index: S2 = Y^T Delta, and per first index a, S3[a] = G_a^T Delta with
// G_a[m][c] = Y_m[a] R_m[c] + X_m[a] Delta_m[c] / 2.
// The chain Delta_{m-1} = P Delta_m keeps row c16 of P in the lane's registers; every lane forms the whole dot
// product from the vector broadcast through LDS, so no cross-lane reduction sits on the chain.
// The wave also writes the interval's flow. LDS per wave: P (256), the vector buffer (32), then one region
// shared by V / scratch (while the step matrices and the flow are formed) and the segment table
// E[m][c] = {Delta, R, Y, X} (row pitch EP floats, MP rows, the rows m >= M zero).
constexpr int EP = 68;  // row pitch of the segment table (four segments of a k-step on distinct banks)

__host__ __device__ constexpr int vl_rows(int M) { return (M + 3) / 4 * 4; }
__host__ __device__ constexpr int vl_region(int M) {
  return 256 + 32 + (EP * vl_rows(M) > 256 + 256 + 32 ? EP * vl_rows(M) : 256 + 256 + 32);
}

__device__ __forceinline__ float dot16(const f4* r, const f4* x) {
  float s0 = r[0].x * x[0].x, s1 = r[0].y * x[0].y, s2 = r[0].z * x[0].z, s3 = r[0].w * x[0].w;
#pragma unroll
  for (int q = 1; q < 4; ++q) {
    s0 = fmaf(r[q].x, x[q].x, s0);
    s1 = fmaf(r[q].y, x[q].y, s1);
    s2 = fmaf(r[q].z, x[q].z, s2);
    s3 = fmaf(r[q].w, x[q].w, s3);
  }
  return (s0 + s1) + (s2 + s3);
}

template <int N, bool EXACTF>  // EXACTF: exact flows (only the scaled exponential is compiled for them)
__global__ __launch_bounds__(256, 2) void k_vl(Args a) {
  extern __shared__ __align__(16) float lds[];
  LdsTable* sp = reinterpret_cast<LdsTable*>(lds);
  const int tid = threadIdx.x, w = tid >> 6, l = tid & 63, g = l >> 4, c16 = l & 15;
  const int nw = blockDim.x >> 6;
  const int Mv = a.vm, MP = vl_rows(Mv);
  stage_lds(lds, a.apow, (PM + 1) * 256, tid, blockDim.x);
  const float norm1 = a.apow[a.npow * 256];
  float* P = lds + (PM + 1) * 256 + w * vl_region(Mv);
  float* xs = P + 256;
  float* V = xs + 32;
  float* T = V + 256;
  float* E = V;
  __syncthreads();
  const long total = (long)a.B * a.n_int;
  // the interval's clock values and increment coordinates are loaded one interval ahead into registers, so that no
  // memory round trip sits at the top of an interval
  const long first = (long)blockIdx.x * nw + w, stride = (long)gridDim.x * nw;
  float nth0 = 0.0f, nth1 = 0.0f, nx0 = 0.0f, nx1 = 0.0f;
  const bool xl = l < 16 && l < a.d;
  auto prefetch = [&](long i2) {
    const int b2 = (int)(i2 / a.n_int), t2 = (int)(i2 - (long)b2 * a.n_int);
    const float* th2 = a.clock + (size_t)b2 * a.L + t2;
    nth0 = th2[0];
    nth1 = th2[1];
    if (xl) {
      const float* x = a.path + ((size_t)b2 * a.L + t2) * a.d;
      nx0 = x[l];
      nx1 = x[a.d + l];
    }
  };
  if (first < total) prefetch(first);
  for (long it = first; it < total; it += stride) {
    const int b = (int)(it / a.n_int), t = (int)(it - (long)b * a.n_int);
    const float* th = a.clock + (size_t)b * a.L;
    const float hi = nth1 - nth0, x0 = nx0, x1 = nx1;  // th[t + 1] - th[t]; path[t][l], path[t + 1][l]
    if (it + stride < total) prefetch(it + stride);
    wave_order_d();  // the previous interval's reads of the segment table come first
    if constexpr (EXACTF) {
      bool ident = false;
      const float hf = a.flow_mode == EWS_FLOW_PER_INTERVAL ? hi : flow_step(a, th, t, ident);
      f4 m;
      if (ident) {
#pragma unroll
        for (int r = 0; r < 4; ++r) m[r] = ((4 * l + r) >> 4) == ((4 * l + r) & 15) ? 1.0f : 0.0f;
      } else if (a.flow_mode != EWS_FLOW_PER_INTERVAL) {
        m = *reinterpret_cast<const f4*>(a.mats + (size_t)b * 768 + 512 + 4 * l);
      } else {
        wave_expm(sp, norm1, hf, P, nullptr, l);
        m = *reinterpret_cast<const f4*>(P + 4 * l);
        wave_order_d();
      }
      *reinterpret_cast<f4*>(a.fl + ((size_t)b * a.n_int + t) * 256 + 4 * l) = m;
    } else {
      write_flow(a, sp, norm1, b, t, th, P, T, l);
    }
    // step matrices
    if (a.vl_mode == EWS_FLOW_PER_INTERVAL) {
      wave_matfn(sp, norm1, a.vl_expm, hi / (float)Mv, false, P, V, T, l);
    } else if (a.vl_mode == EWS_FLOW_CACHED_BASEPOINT && t == 0) {
      wave_identity(P, l);
      wave_identity(V, l);
    } else {
      const float* mb = a.mats + (size_t)b * 768;
      *reinterpret_cast<f4*>(P + 4 * l) = *reinterpret_cast<const f4*>(mb + 4 * l);
      *reinterpret_cast<f4*>(V + 4 * l) = *reinterpret_cast<const f4*>(mb + 256 + 4 * l);
      wave_order_d();
    }
    f4 pr[4], vr[4], xv[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      pr[q] = *reinterpret_cast<const f4*>(P + c16 * 16 + 4 * q);
      vr[q] = *reinterpret_cast<const f4*>(V + c16 * 16 + 4 * q);
    }
    float* sv = a.vlsave ? a.vlsave + ((size_t)b * a.n_int + t) * (512 + 16 * Mv) : nullptr;
    if (sv) {
      *reinterpret_cast<f4*>(sv + 4 * l) = *reinterpret_cast<const f4*>(P + 4 * l);
      *reinterpret_cast<f4*>(sv + 256 + 4 * l) = *reinterpret_cast<const f4*>(V + 4 * l);
    }
    // w = v / M
    if (l < 16) xs[l] = xl ? (x1 - x0) / (float)Mv : 0.0f;
    wave_order_d();
#pragma unroll
    for (int q = 0; q < 4; ++q) xv[q] = *reinterpret_cast<const f4*>(xs + 4 * q);
    float dl = dot16(vr, xv);
    wave_order_d();  // V and the vector are read before they are overwritten
    // rows M .. MP-1 of the table are zero
    for (int e = l; e < (MP - Mv) * 16; e += 64)
      *reinterpret_cast<f4*>(E + (Mv + (e >> 4)) * EP + 4 * (e & 15)) = f4{0.0f, 0.0f, 0.0f, 0.0f};
    // Delta_{M-1} .. Delta_0 (segments indexed from 0) and the suffix sums
    float suf = 0.0f;
    for (int m = Mv - 1;; --m) {
      if (g == 0) *reinterpret_cast<float2*>(E + m * EP + 4 * c16) = float2{dl, suf};
      if (sv && g == 1) sv[512 + m * 16 + c16] = dl;
      suf += dl;
      if (m == 0) break;
      if (g == 0) xs[c16] = dl;
      wave_order_d();
#pragma unroll
      for (int q = 0; q < 4; ++q) xv[q] = *reinterpret_cast<const f4*>(xs + 4 * q);
      wave_order_d();
      dl = dot16(pr, xv);
    }
    float* row = a.loc + ((size_t)b * a.n_int + t) * a.LW;
    if (g == 0) row[c16] = suf;
    wave_order_d();
    // Y and X from Pre_m = S1 - R_m - Delta_m, segments m = g, g + 4, ...
    for (int m = g; m < Mv; m += 4) {
      const float2 dr = *reinterpret_cast<const float2*>(E + m * EP + 4 * c16);
      const float pre = suf - dr.y - dr.x;
      *reinterpret_cast<float2*>(E + m * EP + 4 * c16 + 2) =
          float2{fmaf(0.5f, dr.x, pre), fmaf(1.0f / 3.0f, dr.x, pre)};
    }
    wave_order_d();
    if constexpr (N >= 2) {
      f4 acc2 = {0.0f, 0.0f, 0.0f, 0.0f};
      f4 acc3[N == 3 ? 16 : 1];
#pragma unroll
      for (int i = 0; i < (N == 3 ? 16 : 1); ++i) acc3[i] = f4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll 1
      for (int s = 0; s < MP / 4; ++s) {
        const float* er = E + (4 * s + g) * EP;
        const f4 e = *reinterpret_cast<const f4*>(er + 4 * c16);  // {Delta, R, Y, X}[c16] of segment 4s + g
        acc2 = mfma(e.z, e.x, acc2);
        if constexpr (N == 3) {
          const float hv = 0.5f * e.x;
#pragma unroll
          for (int aa = 0; aa < 16; ++aa) {
            const float2 yx = *reinterpret_cast<const float2*>(er + 4 * aa + 2);  // Y_m[a], X_m[a]
            acc3[aa] = mfma(fmaf(yx.x, e.y, yx.y * hv), e.x, acc3[aa]);
          }
        }
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) row[16 + (4 * g + r) * 16 + c16] = acc2[r];
      if constexpr (N == 3) {
#pragma unroll
        for (int aa = 0; aa < 16; ++aa)
          *reinterpret_cast<f4*>(row + 272 + aa * 256 + c16 * 16 + 4 * g) = acc3[aa];
      }
    }
  }
}

// ------------------------------------------------------------------------------------------------ Chen scan
__device__ __forceinline__ long out_index(int N, int d, int e) {  // padded state index -> unpadded row index
  if (e < 16) return e < d ? e : -1;
  if (N >= 2 && e < 272) {
    const int f = e - 16, i = f >> 4, j = f & 15;
    return (i < d && j < d) ? d + i * d + j : -1;
  }
  const int f = e - 272, i = f >> 8, j = (f >> 4) & 15, k = f & 15;
  return (i < d && j < d && k < d) ? d + d * d + (i * d + j) * d + k : -1;
}
__device__ __forceinline__ void put(const Seq& s, float* orow, int N, int e, float v) {
  if (s.padded || s.d == 16) {  // d = 16: the unpadded row index is the padded one
    orow[e] = v;
  } else {
    const long o = out_index(N, s.d, e);
    if (o >= 0) orow[o] = v;
  }
}

// x through an empty asm statement in a vector register: the compiler can neither fold it nor hoist what is
// computed from it out of the enclosing loop
__device__ __forceinline__ int opaque_vgpr(int x) {
  asm volatile("" : "+v"(x));
  return x;
}
// Operands of one step: the flow as the lane's M[l%16][4g..4g+3], level-1/2 local terms, and the lane's
// level-3 local terms of the output tiles of this wave (j = 4w + jj).
template <int N> struct StepIn {
  f4 M4;
  float s1k;
  f4 s2r;
  f4 s3r[N >= 3 ? 4 : 1];
};
template <int N>
__device__ __forceinline__ void load_step(const Seq& s, int b, int t, int w, int g, int c16, StepIn<N>& in) {
  constexpr int LW = lw_of(N);
  const float* lrow = s.lv + b * s.lv_bs + (long)t * LW;
  const float* frow = s.fl + b * s.fl_bs + (long)t * 256;
  in.M4 = *reinterpret_cast<const f4*>(frow + c16 * 16 + 4 * g);
  in.s1k = lrow[c16];
  if constexpr (N >= 2) {
#pragma unroll
    for (int r = 0; r < 4; ++r) in.s2r[r] = lrow[16 + (4 * g + r) * 16 + c16];
  }
  if constexpr (N >= 3) {
#pragma unroll
    for (int jj = 0; jj < 4; ++jj)
#pragma unroll
      for (int r = 0; r < 4; ++r) in.s3r[jj][r] = lrow[272 + (4 * g + r) * 256 + (4 * w + jj) * 16 + c16];
  }
}

template <int N, bool SUMMARY>
__global__ __launch_bounds__(N >= 3 ? 256 : 64) void k_scan(Seq s) {
  constexpr int LW = lw_of(N);
  __shared__ __align__(16) float s3[N >= 3 ? 16 * SP : 4];
  __shared__ __align__(16) float y3[N >= 3 ? 16 * SP : 4];
  __shared__ __align__(16) float s2[16 * RP];
  __shared__ __align__(16) float s1[16];
  const int tid = threadIdx.x, w = tid >> 6, l = tid & 63, g = l >> 4, c16 = l & 15;
  const int c = blockIdx.x, b = blockIdx.y;
  const int t0 = c * s.T, Tc = min(s.T, s.n - t0);
  const float* ini = s.init ? s.init + b * s.init_bs + (long)c * LW : nullptr;
  if (tid < 16) s1[tid] = ini ? ini[tid] : 0.0f;
  if constexpr (N >= 2) {
    for (int e = tid; e < 256; e += blockDim.x) s2[(e >> 4) * RP + (e & 15)] = ini ? ini[16 + e] : 0.0f;
  }
  if constexpr (N >= 3) {
    for (int e = tid; e < 4096; e += blockDim.x)
      s3[(e >> 8) * SP + ((e >> 4) & 15) * RP + (e & 15)] = ini ? ini[272 + e] : 0.0f;
  }
  // chunk flow product (SUMMARY): result layout, lane holds Mc[4g + r][c16]
  constexpr int WL1 = N >= 3 ? 1 : 0, WMC = N >= 3 ? 2 : 0;
  f4 Mc;
#pragma unroll
  for (int r = 0; r < 4; ++r) Mc[r] = (4 * g + r == c16) ? 1.0f : 0.0f;
  __syncthreads();
  StepIn<N> cur, nxt;
  if (Tc > 0) load_step<N>(s, b, t0, w, g, c16, cur);
  float* orow0 = s.rows ? s.rows + b * s.rows_bs + (long)t0 * s.rows_ld : nullptr;
  for (int t = 0; t < Tc; ++t) {
    if (t + 1 < Tc) load_step<N>(s, b, t0 + t + 1, w, g, c16, nxt);
    const f4 M4 = cur.M4;
    // ---------------- phase A: modes 3 and 2 of level 3 (slices i = 4w + ii), level 2 (wave 0), level 1
    if constexpr (N >= 3) {
#pragma unroll
      for (int ii = 0; ii < 4; ++ii) {
        const int i = 4 * w + ii;
        const f4 A4 = *reinterpret_cast<const f4*>(s3 + i * SP + c16 * RP + 4 * g);  // S3[i][c16][4g + s]
        f4 x = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int k = 0; k < 4; ++k) x = mfma(A4[k], M4[k], x);  // X[i][4g + r][c16] = sum_k S3[i][.][k] M[c16][k]
        const f4 S2i = *reinterpret_cast<const f4*>(s2 + i * RP + 4 * g);
#pragma unroll
        for (int r = 0; r < 4; ++r) x[r] = fmaf(S2i[r], cur.s1k, x[r]);  // + S2[i][4g + r] s1[c16]
        f4 y = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int r = 0; r < 4; ++r) y = mfma(M4[r], x[r], y);  // Y[i][4g + r][c16] = sum_j M[.][j] X[i][j][c16]
        const float S1i = s1[i];
#pragma unroll
        for (int r = 0; r < 4; ++r) y3[i * SP + (4 * g + r) * RP + c16] = fmaf(S1i, cur.s2r[r], y[r]);
      }
    }
    f4 n2 = {0.0f, 0.0f, 0.0f, 0.0f};
    if constexpr (N >= 2) {
      if (w == 0) {
        const f4 A4 = *reinterpret_cast<const f4*>(s2 + c16 * RP + 4 * g);  // S2[c16][4g + s]
        f4 x = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int k = 0; k < 4; ++k) x = mfma(A4[k], M4[k], x);  // (S2 M^T)[4g + r][c16]
        const f4 S1g = *reinterpret_cast<const f4*>(s1 + 4 * g);
#pragma unroll
        for (int r = 0; r < 4; ++r) x[r] = fmaf(S1g[r], cur.s1k, x[r]);  // + S1[4g + r] s1[c16]
#pragma unroll
        for (int r = 0; r < 4; ++r) n2 = mfma(M4[r], x[r], n2);  // M (.) : S2'[4g + r][c16] - s2
#pragma unroll
        for (int r = 0; r < 4; ++r) n2[r] += cur.s2r[r];
      }
    }
    float n1 = 0.0f;
    if (w == WL1) {
      const f4 S1g = *reinterpret_cast<const f4*>(s1 + 4 * g);
      float part = 0.0f;
#pragma unroll
      for (int r = 0; r < 4; ++r) part = fmaf(M4[r], S1g[r], part);  // sum over j = 4g + r of M[c16][j] S1[j]
      part = lanes::add_xor32(lanes::add_xor16(part));
      n1 = part + cur.s1k;
    }
    if constexpr (SUMMARY) {
      if (w == WMC) {
        f4 m = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int r = 0; r < 4; ++r) m = mfma(M4[r], Mc[r], m);  // M_t Mc
        Mc = m;
      }
    }
    __syncthreads();
    // ---------------- phase B: mode 1 of level 3 (tiles j = 4w + jj), write the new state
    float* orow = (!SUMMARY && orow0) ? orow0 + (long)t * s.rows_ld : nullptr;
    if (orow && s.lvl0 && tid == 0) orow[0] = 1.0f;
    float* orl = orow ? orow + s.lvl0 : nullptr;
    if constexpr (N >= 3) {
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        const int j = 4 * w + jj;
        f4 z = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int k = 0; k < 4; ++k) z = mfma(M4[k], y3[(4 * g + k) * SP + j * RP + c16], z);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float v = z[r] + cur.s3r[jj][r];
          s3[(4 * g + r) * SP + j * RP + c16] = v;
          if (orl) put(s, orl, N, 272 + (4 * g + r) * 256 + j * 16 + c16, v);
        }
      }
    }
    if constexpr (N >= 2) {
      if (w == 0) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          s2[(4 * g + r) * RP + c16] = n2[r];
          if (orl) put(s, orl, N, 16 + (4 * g + r) * 16 + c16, n2[r]);
        }
      }
    }
    if (w == WL1 && l < 16) {
      s1[c16] = n1;
      if (orl) put(s, orl, N, c16, n1);
    }
    __syncthreads();
    cur = nxt;
  }
  if constexpr (SUMMARY) {
    float* so = s.summ + ((long)b * s.C + c) * LW;
    for (int e = tid; e < LW; e += blockDim.x) {
      float v;
      if (e < 16) v = s1[e];
      else if (e < 272) v = s2[((e - 16) >> 4) * RP + ((e - 16) & 15)];
      else {
        const int f = e - 272;
        v = s3[(f >> 8) * SP + ((f >> 4) & 15) * RP + (f & 15)];
      }
      so[e] = v;
    }
    if (w == WMC) {
      float* mo = s.sfl + ((long)b * s.C + c) * 256;
#pragma unroll
      for (int r = 0; r < 4; ++r) mo[(4 * g + r) * 16 + c16] = Mc[r];
    }
  }
}

// ------------------------------------------------------------------------------------------------ adjoint scan
// Reverse mode of the Chen scan (the chunked design of pallas_combine.py:1425-1436; the dense kernel's VJP
// _dense_kernel_general_bwd, pallas_combine.py:2360-2565). The step S_t = R_t(S_{t-1}) = (M_t . S_{t-1}) (x) s_t is
// affine in S, so with lambda_t the cotangent of S_t and g_t the readout's cotangent of row t
//   lambda_{t-1} = g_{t-1} + R_t^T lambda_t,
//   R_t^T l = (M^T rho_1, M^T rho_2 M, rho_3 x_1 M^T x_2 M^T x_3 M^T),
//   rho_1 = l_1 + l_2 ._2 s1 + l_3 ._23 s2,   rho_2 = l_2 + l_3 ._3 s1,   rho_3 = l_3.
// The cotangents of the step's inputs (EMIT), with y1 = M S1 and Y2 = M S2 M^T of the state before the step:
//   ds3 = l_3,   ds2 = l_2 + y1 ._1 l_3,   ds1 = l_1 + y1 ._1 l_2 + Y2 ._12 l_3,
//   dM = rho_1 (x) S1 + rho_2 M S2^T + rho_2^T M S2 + T1 + T2 + T3,
// where T1 + T2 + T3 is the derivative of <l_3, M^(x)3 S3> along each tensor axis:
//   T1 = <l_3 x_3 M^T x_2 M^T, S3>_{23},  T2 = <l_3 x_3 M^T, S3 x_1 M>_{13},  T3 = <l_3, S3 x_1 M x_2 M>_{12}
// (<X, Y>_{jk}[p][q] contracts the two named axes of X[.., p, ..] and Y[.., q, ..]). S3 of the state is read from
// its row in global memory (L2-resident), which keeps the workgroup within half of the LDS.
// Passes: LOCAL (each chunk from lambda = 0: the chunk's own part of the cotangent of its entry state),
// CARRY (one sample's chunks in reverse, on the chunk summaries: Lambda_c = local_c + R(chunk c)^T Lambda_{c+1}),
// EMIT (each chunk from Lambda_{c+1}, writing ds_t over the local terms and dM_t over the flows).
// Mode products and the T contractions are 16x16x4 float32 MFMAs (operand conventions as in k_scan).
enum { ADJ_LOCAL = 0, ADJ_CARRY = 1, ADJ_EMIT = 2 };
enum { G_NONE = 0, G_PREFIX = 1, G_MEAN = 2, G_MAX = 3 };

struct AdjSeq {
  const float* lv;  // local terms (padded, LW per row) or chunk summaries (CARRY)
  long lv_bs;
  const float* fl;  // flows (256 per row) or chunk flow products
  long fl_bs;
  int n, T, C, d;
  // readout cotangent of row t: G_PREFIX rows (B, n, W) (glvl0: with the level-0 column); G_MEAN one row (B, W)
  // scaled by gscale; G_MAX one row (B, W) applied where amax == t
  int gmode, W, glvl0;
  const float* g;
  const int* amax;
  float gscale;
  const float* init;  // EMIT: Lambda rows (B, C + 1, LW), chunk c starts from row c + 1
  float* lam;         // LOCAL: (B, C, LW) outputs
  const float* lloc;  // CARRY: the local parts, row t at lloc + b * lloc_bs + t * LW
  // CARRY: workgroup c takes rows [c T, min(c T + T, n)) in reverse, from the row init + b * init_bs +
  // (c + init_off) * LW (zero when init is null); before row t it writes lambda to row t + 1 of lam (lam_bs per
  // sample) when lam is set and t + 1 < lam_lim, and at the end the workgroup's lambda to row c of agg (agg_bs)
  long init_bs, lloc_bs, lam_bs, agg_bs;
  int init_off, lam_lim;
  float* agg;
  const float* st;    // EMIT: the states S_t, padded rows (B, n, st_ld floats apart; st_ld >= LW)
  long st_ld;
  float* dlv;         // EMIT: ds_t (padded, in place of lv)
  float* dfl;         // EMIT: dM_t (in place of fl)
};

__device__ __forceinline__ float adj_g(const AdjSeq& s, int b, int t, int e, int N) {
  if (s.gmode == G_NONE) return 0.0f;
  const long oi = out_index(N, s.d, e);
  if (oi < 0) return 0.0f;
  const long col = s.glvl0 + oi;
  if (s.gmode == G_PREFIX) return s.g[((long)b * s.n + t) * s.W + col];
  if (s.gmode == G_MEAN) return s.g[(long)b * s.W + col] * s.gscale;
  return s.amax[(long)b * LWN(N) + e] == t ? s.g[(long)b * s.W + col] : 0.0f;
}

// The inputs of one adjoint step of thread tid: the flow entry M[tid / 16][tid % 16], the local terms' level 1
// (tid < 16) and level-2 entry tid, the row added this step (entries tid, 16 + tid and the sixteen level-3 entries
// 272 + 16 tid + i: the readout cotangent g_t, or for CARRY the chunk's local part), and for EMIT the state before
// the step (levels 1-2).
// LDS row of 16 floats (16-byte aligned) += v
__device__ __forceinline__ void add_row16(float* row, const float* v) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f4 x = *reinterpret_cast<const f4*>(row + 4 * i);
#pragma unroll
    for (int r = 0; r < 4; ++r) x[r] += v[4 * i + r];
    *reinterpret_cast<f4*>(row + 4 * i) = x;
  }
}
template <int N, int MODE> struct AdjIn {
  float M, s1, s2, r1, r2;
  float r3[N >= 3 ? 16 : 1];
  float S1, S2;
};
template <int N, int MODE>
__device__ __forceinline__ void adj_load(const AdjSeq& s, int b, int t, int tid, AdjIn<N, MODE>& x) {
  constexpr int LW = lw_of(N);
  const float* lrow = s.lv + b * s.lv_bs + (long)t * LW;
  const float* frow = s.fl + b * s.fl_bs + (long)t * 256;
  x.M = frow[tid];
  x.s1 = tid < 16 ? lrow[tid] : 0.0f;
  if constexpr (N >= 2) x.s2 = lrow[16 + tid];
  x.r1 = x.r2 = 0.0f;
#pragma unroll
  for (int i = 0; i < (N >= 3 ? 16 : 1); ++i) x.r3[i] = 0.0f;
  if constexpr (MODE == ADJ_CARRY) {
    const float* lo = s.lloc + b * s.lloc_bs + (long)t * LW;
    if (tid < 16) x.r1 = lo[tid];
    if constexpr (N >= 2) x.r2 = lo[16 + tid];
    if constexpr (N >= 3) {
      const f4* q = reinterpret_cast<const f4*>(lo + 272 + 16 * tid);  // rows of LW floats: 16-byte aligned
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const f4 v = q[i];
#pragma unroll
        for (int r = 0; r < 4; ++r) x.r3[4 * i + r] = v[r];
      }
    }
  } else if (s.gmode == G_PREFIX && s.d == 16) {  // unpadded rows: the cotangent row is the state layout
    const float* grow = s.g + ((long)b * s.n + t) * s.W + s.glvl0;
    if (tid < 16) x.r1 = grow[tid];
    if constexpr (N >= 2) x.r2 = grow[16 + tid];
    if constexpr (N >= 3) {
      const float* q = grow + 272 + 16 * tid;  // any alignment (rows of W floats)
#pragma unroll
      for (int i = 0; i < 16; ++i) x.r3[i] = q[i];
    }
  }  // the other readouts' cotangents (index mapping, mean, max) are read inside the step
  x.S1 = x.S2 = 0.0f;
  if constexpr (MODE == ADJ_EMIT) {
    if (t > 0) {
      const float* srow = s.st + ((long)b * s.n + t - 1) * s.st_ld;
      if (tid < 16) x.S1 = srow[tid];
      if constexpr (N >= 2) x.S2 = srow[16 + tid];
    }
  }
}

template <int N, int MODE>
__global__ __launch_bounds__(256, 2) void k_adj(AdjSeq s) {
  constexpr int LW = lw_of(N);
  constexpr bool EMIT = MODE == ADJ_EMIT;
  constexpr int S3N = N >= 3 ? 16 * SP : 4;
  __shared__ __align__(16) float L3[S3N];                  // l_3 (current cotangent, level 3)
  __shared__ __align__(16) float C3[S3N];                  // l_3 x_3 M^T, then x_2 M^T
  __shared__ __align__(16) float B3[EMIT ? S3N : 4];       // S3 x_1 M, then x_2 M
  __shared__ __align__(16) float Tw[EMIT && N >= 3 ? 4 : 1][256];  // per-wave partial T1 + T2 + T3
  __shared__ __align__(16) float L2[16 * RP], R2[16 * RP], Ms[256], s2s[16 * RP], Zs[16 * RP];
  __shared__ __align__(16) float S2s[16 * RP], MS2[16 * RP], MS2T[16 * RP], Y2s[16 * RP], Qs[16 * RP];
  __shared__ float L1[16], R1[16], s1s[16], S1s[16], y1s[16];
  const int tid = threadIdx.x, w = tid >> 6, l = tid & 63, g = l >> 4, c16 = l & 15;
  const int ri = tid >> 4, rj = tid & 15;  // (row, column) of the 16 x 16 VALU work
  const int b = blockIdx.y;
  const int c = blockIdx.x, t0 = c * s.T, Tc = min(s.T, s.n - t0);
  // initial lambda
  {
    const float* ini = nullptr;
    if constexpr (MODE == ADJ_EMIT) ini = s.init + ((long)b * (s.C + 1) + c + 1) * LW;
    if constexpr (MODE == ADJ_CARRY) ini = s.init ? s.init + b * s.init_bs + (long)(c + s.init_off) * LW : nullptr;
    if (tid < 16) L1[tid] = ini ? ini[tid] : 0.0f;
    if constexpr (N >= 2) L2[ri * RP + rj] = ini ? ini[16 + tid] : 0.0f;
    if constexpr (N >= 3) {
      for (int e = tid; e < 4096; e += 256) L3[(e >> 8) * SP + ((e >> 4) & 15) * RP + (e & 15)] = ini ? ini[272 + e] : 0.0f;
    }
  }
  __syncthreads();
  // The inputs of step t are loaded one step ahead into registers (cur / nxt), so that no global load sits on the
  // step's dependency chain: the flow, the local terms' levels 1-2, the row added this step (the readout's
  // cotangent row g_t, or CARRY's local part, added at the end of the step), and for EMIT the state before the step.
  AdjIn<N, MODE> cur, nxt;
  if (Tc > 0) adj_load<N, MODE>(s, b, t0 + Tc - 1, tid, cur);
  const int tid_all = tid;
  for (int k = Tc - 1; k >= 0; --k) {
    const int t = t0 + k;  // row (interval / chunk) index
    // the lane indices are re-derived every step from an opaque copy of the thread index, so that the compiler
    // recomputes the step's LDS and global addresses (a few integer instructions) instead of keeping every one of
    // them live across the loop
    const int tid = opaque_vgpr(tid_all), w = tid >> 6, l = tid & 63, g = l >> 4, c16 = l & 15;
    const int ri = tid >> 4, rj = tid & 15;
    (void)l;
    // CARRY stores a row every step: the next step's inputs are issued before it, since the memory counter is in
    // order and a load issued after a store is waited for together with the store
    if (MODE == ADJ_CARRY && k > 0) adj_load<N, MODE>(s, b, t - 1, tid, nxt);
    if constexpr (MODE == ADJ_CARRY) {  // Lambda_{t+1} is the current lambda
      float* o = s.lam + b * s.lam_bs + (long)(t + 1) * LW;
      if (s.lam && t + 1 < s.lam_lim) {
        if (tid < 16) o[tid] = L1[tid];
        if constexpr (N >= 2) o[16 + tid] = L2[ri * RP + rj];
        if constexpr (N >= 3) {
          const float* src = L3 + (tid >> 4) * SP + (tid & 15) * RP;
          f4* dst = reinterpret_cast<f4*>(o + 272 + 16 * tid);
#pragma unroll
          for (int i = 0; i < 4; ++i) dst[i] = *reinterpret_cast<const f4*>(src + 4 * i);
        }
      }
    }
    // ---- inputs of the step; lambda += g_t
    Ms[tid] = cur.M;
    if (tid < 16) s1s[tid] = cur.s1;
    if constexpr (N >= 2) s2s[ri * RP + rj] = cur.s2;
    if constexpr (MODE != ADJ_CARRY) {
      if (s.gmode == G_PREFIX && s.d == 16) {
        if (tid < 16) L1[tid] += cur.r1;
        if constexpr (N >= 2) L2[ri * RP + rj] += cur.r2;
        if constexpr (N >= 3) add_row16(L3 + (tid >> 4) * SP + (tid & 15) * RP, cur.r3);
      } else if (s.gmode != G_NONE) {
        if (tid < 16) L1[tid] += adj_g(s, b, t, tid, N);
        if constexpr (N >= 2) L2[ri * RP + rj] += adj_g(s, b, t, 16 + tid, N);
        if constexpr (N >= 3) {
          for (int e = tid; e < 4096; e += 256)
            L3[(e >> 8) * SP + ((e >> 4) & 15) * RP + (e & 15)] += adj_g(s, b, t, 272 + e, N);
        }
      }
    }
    if constexpr (EMIT) {  // the state before the step (zero before the first interval)
      if (tid < 16) S1s[tid] = cur.S1;
      if constexpr (N >= 2) S2s[ri * RP + rj] = cur.S2;
    }
    // EMIT, depth 3: the lane's operands of S3 (state before the step) for V1 = S3 x_1 M (s3v) and for T1 (s3t),
    // issued before the next step's inputs so that their wait does not cover those
    constexpr int NS3 = EMIT && N >= 3 ? 16 : 1;
    float s3v[NS3], s3t[NS3];
    if constexpr (EMIT && N >= 3) {
      const float* s3g = t > 0 ? s.st + ((long)b * s.n + t - 1) * s.st_ld + 272 : nullptr;
      // S3[4g + k2][4w + jj][c16] and S3[c16][4w + q / 4][4 (q % 4) + g]: one base each, offsets within 4 KB
      const float* pv = s3g + (4 * g * 256 + 4 * w * 16 + c16);
      const float* pt = s3g + (c16 * 256 + 4 * w * 16 + g);
#pragma unroll
      for (int jj = 0; jj < 4; ++jj)
#pragma unroll
        for (int k2 = 0; k2 < 4; ++k2) s3v[4 * jj + k2] = s3g ? pv[k2 * 256 + jj * 16] : 0.0f;
#pragma unroll
      for (int q = 0; q < 16; ++q) s3t[q] = s3g ? pt[(q >> 2) * 16 + 4 * (q & 3)] : 0.0f;
    }
    if (MODE != ADJ_CARRY && k > 0) adj_load<N, MODE>(s, b, t - 1, tid, nxt);  // the next step's inputs
    __syncthreads();
    const f4 M4 = *reinterpret_cast<const f4*>(Ms + c16 * 16 + 4 * g);  // M[c16][4g + r]
    f4 MT4;                                                                // M^T[c16][4g + r]
#pragma unroll
    for (int r = 0; r < 4; ++r) MT4[r] = Ms[(4 * g + r) * 16 + c16];
    float* drow = EMIT ? s.dlv + b * s.lv_bs + (long)t * LW : nullptr;
    // ---- rho_2, rho_1 (and for EMIT y1, M S2, M S2^T, ds3)
    {
      float r2 = 0.0f, pp = 0.0f;
      if constexpr (N >= 3) {
        const float* row = L3 + ri * SP + rj * RP;  // l_3[ri][rj][.]
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const f4 x = *reinterpret_cast<const f4*>(row + 4 * q);
          const f4 a1 = *reinterpret_cast<const f4*>(s1s + 4 * q);
          const f4 a2 = *reinterpret_cast<const f4*>(s2s + rj * RP + 4 * q);
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            r2 = fmaf(x[r], a1[r], r2);
            pp = fmaf(x[r], a2[r], pp);
          }
        }
      }
      float v = pp;
      if constexpr (N >= 2) {
        const float l2 = L2[ri * RP + rj];
        R2[ri * RP + rj] = l2 + r2;
        v = fmaf(l2, s1s[rj], v);
      }
      v = lanes::sum16(v);
      if (rj == 0) R1[ri] = L1[ri] + v;
      if constexpr (EMIT) {
        float m = Ms[ri * 16 + rj] * S1s[rj];
        m = lanes::sum16(m);
        if (rj == 0) y1s[ri] = m;
        if constexpr (N >= 2) {
          float a = 0.0f, bt = 0.0f;
#pragma unroll
          for (int k2 = 0; k2 < 16; ++k2) {
            const float mik = Ms[ri * 16 + k2];
            a = fmaf(mik, S2s[k2 * RP + rj], a);   // (M S2)[ri][rj]
            bt = fmaf(mik, S2s[rj * RP + k2], bt);  // (M S2^T)[ri][rj]
          }
          MS2[ri * RP + rj] = a;
          MS2T[ri * RP + rj] = bt;
        }
      }
    }
    __syncthreads();
    // ---- EMIT: Y2 = (M S2) M^T, dM of levels 1-2, ds2
    float dm12 = 0.0f;
    if constexpr (EMIT) {
      if constexpr (N >= 2) {
        float y = 0.0f;
#pragma unroll
        for (int k2 = 0; k2 < 16; ++k2) y = fmaf(MS2[ri * RP + k2], Ms[rj * 16 + k2], y);
        Y2s[ri * RP + rj] = y;
      }
      dm12 = R1[ri] * S1s[rj];
      if constexpr (N >= 2) {
#pragma unroll
        for (int k2 = 0; k2 < 16; ++k2) {
          dm12 = fmaf(R2[ri * RP + k2], MS2T[k2 * RP + rj], dm12);
          dm12 = fmaf(R2[k2 * RP + ri], MS2[k2 * RP + rj], dm12);
        }
      }
    }
    __syncthreads();
    float ds2v = 0.0f;
    if constexpr (EMIT) {
      if constexpr (N >= 2) {
        // ds2[ri][rj] = l_2[ri][rj] + sum_a y1[a] l_3[a][ri][rj];  Q[ri][rj] = sum_a l_3[a][ri][rj] Y2[a][ri]
        ds2v = L2[ri * RP + rj];
        float qv = 0.0f;
        if constexpr (N >= 3) {
#pragma unroll
          for (int a = 0; a < 16; ++a) {
            const float x = L3[a * SP + ri * RP + rj];
            ds2v = fmaf(y1s[a], x, ds2v);
            qv = fmaf(Y2s[a * RP + ri], x, qv);
          }
        }
        // ds1[rj] = l_1[rj] + sum_a l_2[a][rj] y1[a] + sum_ri Q[ri][rj]
        Qs[ri * RP + rj] = qv + L2[ri * RP + rj] * y1s[ri];
      }
    }
    // ---- level-3 mode products and the T contractions
    f4 tacc = {0.0f, 0.0f, 0.0f, 0.0f};
    if constexpr (N >= 3) {
      f4 a23[4];
#pragma unroll
      for (int ii = 0; ii < 4; ++ii) {
        const int i = 4 * w + ii;
        const f4 A4 = *reinterpret_cast<const f4*>(L3 + i * SP + c16 * RP + 4 * g);  // l_3[i][c16][4g + k]
        f4 x = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int k2 = 0; k2 < 4; ++k2) x = mfma(A4[k2], MT4[k2], x);  // (l_3 x_3 M^T)[i][4g + r][c16]
#pragma unroll
        for (int r = 0; r < 4; ++r) C3[i * SP + (4 * g + r) * RP + c16] = x[r];
        f4 y = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int r = 0; r < 4; ++r) y = mfma(MT4[r], x[r], y);  // (.. x_2 M^T)[i][4g + r][c16]
        a23[ii] = y;
      }
      if constexpr (EMIT) {
        // V1 = S3 x_1 M, tiles j, with S3 read from the state row (L2-resident; zero before the first interval)
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
          const int j = 4 * w + jj;
          f4 z = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
          for (int k2 = 0; k2 < 4; ++k2) z = mfma(M4[k2], s3v[4 * jj + k2], z);
#pragma unroll
          for (int r = 0; r < 4; ++r) B3[(4 * g + r) * SP + j * RP + c16] = z[r];
        }
      }
      __syncthreads();
      if constexpr (EMIT) {
        // T2[p][q] = sum_{a, c} C3[a][p][c] V1[a][q][c]; this wave's k-steps 16w .. 16w + 15
#pragma unroll 4
        for (int ks = 16 * w; ks < 16 * w + 16; ++ks) {
          const int a = ks >> 2, cc = 4 * (ks & 3) + g;
          tacc = mfma(C3[a * SP + c16 * RP + cc], B3[a * SP + c16 * RP + cc], tacc);
        }
      }
      __syncthreads();
#pragma unroll
      for (int ii = 0; ii < 4; ++ii) {
        const int i = 4 * w + ii;
#pragma unroll
        for (int r = 0; r < 4; ++r) C3[i * SP + (4 * g + r) * RP + c16] = a23[ii][r];
        if constexpr (EMIT) {  // W3 = V1 x_2 M, slice i in place
          f4 xv;
#pragma unroll
          for (int r = 0; r < 4; ++r) xv[r] = B3[i * SP + (4 * g + r) * RP + c16];
          f4 y = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
          for (int r = 0; r < 4; ++r) y = mfma(M4[r], xv[r], y);
#pragma unroll
          for (int r = 0; r < 4; ++r) B3[i * SP + (4 * g + r) * RP + c16] = y[r];
        }
      }
      __syncthreads();
      if constexpr (EMIT) {
        // T1[p][q] = sum_{j, k} C3[p][j][k] S3[q][j][k];  T3[p][q] = sum_{a, b} l_3[a][b][p] W3[a][b][q]
#pragma unroll
        for (int q = 0; q < 16; ++q) {
          const int ks = 16 * w + q, j = ks >> 2, kk = 4 * (ks & 3) + g;
          tacc = mfma(C3[c16 * SP + j * RP + kk], s3t[q], tacc);
          tacc = mfma(L3[j * SP + kk * RP + c16], B3[j * SP + kk * RP + c16], tacc);
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) Tw[w][(4 * g + r) * 16 + c16] = tacc[r];
        // ds3 = l_3 (the step's cotangent of its level-3 local term); L3 is rewritten after the next barrier
        {
          const float* src = L3 + (tid >> 4) * SP + (tid & 15) * RP;
          f4* dst = reinterpret_cast<f4*>(drow + 272 + 16 * tid);  // padded rows of LW floats: 16-byte aligned
#pragma unroll
          for (int i = 0; i < 4; ++i) dst[i] = *reinterpret_cast<const f4*>(src + 4 * i);
        }
      }
      __syncthreads();
      // l_3 <- C3 x_1 M^T (tiles j)
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        const int j = 4 * w + jj;
        f4 z = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int k2 = 0; k2 < 4; ++k2) z = mfma(MT4[k2], C3[(4 * g + k2) * SP + j * RP + c16], z);
#pragma unroll
        for (int r = 0; r < 4; ++r) L3[(4 * g + r) * SP + j * RP + c16] = z[r];
      }
    }
    // ---- l_2 <- M^T rho_2 M (via Z = rho_2 M), l_1 <- M^T rho_1; EMIT outputs
    if constexpr (N >= 2) {
      float z = 0.0f;
#pragma unroll
      for (int k2 = 0; k2 < 16; ++k2) z = fmaf(R2[ri * RP + k2], Ms[k2 * 16 + rj], z);
      Zs[ri * RP + rj] = z;
    }
    if constexpr (EMIT) {
      float dm = dm12;
      if constexpr (N >= 3) dm += Tw[0][tid] + Tw[1][tid] + Tw[2][tid] + Tw[3][tid];
      s.dfl[b * s.fl_bs + (long)t * 256 + tid] = dm;
      if constexpr (N >= 2) drow[16 + tid] = ds2v;
    }
    __syncthreads();
    if constexpr (N >= 2) {
      float v = 0.0f;
#pragma unroll
      for (int k2 = 0; k2 < 16; ++k2) v = fmaf(Ms[k2 * 16 + ri], Zs[k2 * RP + rj], v);
      L2[ri * RP + rj] = v;
    }
    if (tid < 16) {
      float v = 0.0f;
#pragma unroll
      for (int k2 = 0; k2 < 16; ++k2) v = fmaf(Ms[k2 * 16 + tid], R1[k2], v);
      if constexpr (EMIT) {
        float d1 = L1[tid];
        if constexpr (N >= 2) {
#pragma unroll
          for (int k2 = 0; k2 < 16; ++k2) d1 += Qs[k2 * RP + tid];
        }
        drow[tid] = d1;
      }
      L1[tid] = v;
    }
    if constexpr (MODE == ADJ_CARRY) {  // Lambda_t = R^T Lambda_{t+1} + local_t
      __syncthreads();
      if (tid < 16) L1[tid] += cur.r1;
      if constexpr (N >= 2) L2[ri * RP + rj] += cur.r2;
      if constexpr (N >= 3) add_row16(L3 + (tid >> 4) * SP + (tid & 15) * RP, cur.r3);
    }
    __syncthreads();
    cur = nxt;
  }
  if (MODE == ADJ_LOCAL || (MODE == ADJ_CARRY && s.agg)) {
    float* o = MODE == ADJ_LOCAL ? s.lam + ((long)b * s.C + c) * LW : s.agg + b * s.agg_bs + (long)c * LW;
    if (tid < 16) o[tid] = L1[tid];
    if constexpr (N >= 2) o[16 + tid] = L2[ri * RP + rj];
    if constexpr (N >= 3) {
      for (int e = tid; e < 4096; e += 256) o[272 + e] = L3[(e >> 8) * SP + ((e >> 4) & 15) * RP + (e & 15)];
    }
  }
}

// ------------------------------------------------------------------------------------------------ leaf adjoints
// Cotangents of the leaf and the flows of one interval, given ds_t (the local terms' cotangent, padded) and dM_t,
// one workgroup of 256 threads per interval (grid-stride); thread e owns entry e = 16 i + j of d x d matrices.
// Outputs per interval: dv_t (the increment's cotangent) and dh_t (the clock step's); per sample: the cotangent of
// the shared flow step (cached modes); per workgroup: dA terms.
// dA is collected in two parts. Terms of the recursions b_p = (-h/p) A b_{p-1} go straight to a d x d sum. Terms of
// matrix polynomials in A (the flows' Taylor polynomial T(y) = sum_p (y^p / p!) A^p) collect the cotangent H_p of
// each power A^p; k_dA then forms sum_p sum_{j<p} (A^T)^j H_p (A^T)^{p-1-j} once.
//
// Series leaf (series_leaf.py:55-126 restated as nested degree sums; see k_local): with g1_n = b_n / (n+1),
//   s1 = sum_n g1_n;  s2 = sum_n bt2_n (x) g1_n, bt2_n = sum_{p <= q-n} b_p / (p+n+2);
//   s3 = sum_N bt3_N (x) g2_N, bt3_N = sum_{p <= q-N} b_p / (p+N+3), g2_N = 1/(N+2) sum_{p+n=N} b_p (x) g1_n
//   (and s2 = sum_N g2_N at depth 3).
// Flows (exact): M = T(y)^(2^s), y = -h / 2^s; the squarings' adjoint G <- G E^T + E^T G, then T's.
constexpr int HP = PM + 1;   // powers with a collected cotangent H_p, p <= PM

struct LeafBwd {
  float* dv;    // (B, n, 16)
  float* dh;    // (B, n)
  float* dsh;   // (B, 2): cotangents of the shared flow step and of the shared Van Loan step (cached modes)
  float* dshi;  // (B, n, 2): their per-interval terms, reduced into dsh in a fixed order
  float* part;  // (gridDim.x, HP + 1, 256): per-workgroup H_0..H_PM and the direct dA terms
};

// 1/n for a small positive integer n, by the hardware reciprocal (within 1 ulp; the adjoints' rounding budget)
__device__ __forceinline__ float frcp(int n) { return __builtin_amdgcn_rcpf((float)n); }

// workgroup sum (256 threads) of one value per thread; red: 4 floats of LDS. Every thread gets the sum.
__device__ __forceinline__ float block_sum(float v, float* red, int tid) {
  v = lanes::sum64(v);
  __syncthreads();
  if ((tid & 63) == 0) red[tid >> 6] = v;
  __syncthreads();
  return (red[0] + red[1]) + (red[2] + red[3]);
}

// Adjoint of E = exp(-c A) and Phi = phi(-c A) as the kernels evaluate them (wave_expm / series_mats: Taylor
// polynomials of degree PM in y = -c / 2^s, then s doublings E <- E E, Phi <- (Phi + Phi E) / 2). GE and GPhi
// (GPhi may be null) are the cotangents in LDS, overwritten. Adds the cotangents of the powers A^p to H (entry
// tid) and returns the cotangent of c. Esq, Fsq: SQMAX matrices of LDS each (Fsq unused without GPhi).
__device__ float block_exp_adjoint(const LdsTable* sp, float norm1, float c, float* GE, float* GPhi,
                                   float (*Esq)[256], float (*Fsq)[256], float* red, float* H, int tid) {
  const int i = tid >> 4, j = tid & 15;
  int s = 0;
  float x = fabsf(c) * norm1;
  while (x > 1.0f && s < SQMAX) {
    x *= 0.5f;
    ++s;
  }
  const float y = -c * ldexpf(1.0f, -s);
  float e = sp[PM][tid], f = e * (1.0f / (float)(PM + 1));
#pragma unroll
  for (int p = PM - 1; p >= 0; --p) {
    e = fmaf(e, y, sp[p][tid]);
    f = fmaf(f, y, sp[p][tid] * (1.0f / (float)(p + 1)));
  }
  if (s > 0) {
    Esq[0][tid] = e;
    if (GPhi) Fsq[0][tid] = f;
  }
  __syncthreads();
  for (int r = 1; r < s; ++r) {
    float e2 = 0.0f, f2 = 0.0f;
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      const float ekj = Esq[r - 1][k * 16 + j];
      e2 = fmaf(Esq[r - 1][i * 16 + k], ekj, e2);
      if (GPhi) f2 = fmaf(Fsq[r - 1][i * 16 + k], ekj, f2);
    }
    Esq[r][tid] = e2;
    if (GPhi) Fsq[r][tid] = 0.5f * (Fsq[r - 1][tid] + f2);
    __syncthreads();
  }
  for (int r = s - 1; r >= 0; --r) {
    // E' = E E, Phi' = (Phi + Phi E) / 2:  GE <- GE' E^T + E^T GE' + Phi^T GPhi' / 2,  GPhi <- (GPhi' + GPhi' E^T) / 2
    float ge = 0.0f, gf = 0.0f, gfe = 0.0f;
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      ge = fmaf(GE[i * 16 + k], Esq[r][j * 16 + k], ge);
      ge = fmaf(Esq[r][k * 16 + i], GE[k * 16 + j], ge);
      if (GPhi) {
        gf = fmaf(Fsq[r][k * 16 + i], GPhi[k * 16 + j], gf);
        gfe = fmaf(GPhi[i * 16 + k], Esq[r][j * 16 + k], gfe);
      }
    }
    const float gp = GPhi ? GPhi[tid] : 0.0f;
    __syncthreads();
    GE[tid] = fmaf(0.5f, gf, ge);
    if (GPhi) GPhi[tid] = 0.5f * (gp + gfe);
    __syncthreads();
  }
  const float g0 = GE[tid], p0 = GPhi ? GPhi[tid] : 0.0f;
  float yp = 1.0f, ifact = 1.0f, dy = 0.0f, ypm1 = 1.0f;  // ifact = 1/p! (compile-time constants)
#pragma unroll
  for (int p = 0; p < HP; ++p) {
    if (p) ifact *= 1.0f / (float)p;
    const float gsum = g0 + p0 * (1.0f / (float)(p + 1));
    H[p] = fmaf(yp * ifact, gsum, H[p]);
    if (p) {
      dy = fmaf((float)p * ypm1 * sp[p][tid], gsum, dy);
      ypm1 *= y;
    }
    yp *= y;
  }
  return -block_sum(dy, red, tid) * ldexpf(1.0f, -s);
}

// Adjoint of the rational schemes' matrices (wave_matfn): V = N^{-1}, N = I + alpha A + beta A^2, and P = 2V - I
// (cayley), V (euler), I - c V A (pade), with (alpha, beta) = (c/2, 0), (c, 0), (c/2, c^2/12). V, GP and GV (GV may
// be null) in LDS; dN = -V^T GV' V^T for the total cotangent GV' of V. Adds the direct dA terms to dAl (entry tid)
// and returns the cotangent of c. W1, W2: 256 floats of LDS scratch each.
__device__ float block_rational_adjoint(const LdsTable* sp, int scheme, float c, const float* V, const float* GP,
                                        const float* GV, float* W1, float* W2, float* red, float& dAl, int tid) {
  const int i = tid >> 4, j = tid & 15;
  const float* A = sp[1];
  float gv = GV ? GV[tid] : 0.0f, dc = 0.0f;
  if (scheme == EWS_EXPM_CAYLEY) gv = fmaf(2.0f, GP[tid], gv);
  else if (scheme == EWS_EXPM_EULER) gv += GP[tid];
  else {  // pade: P = I - c V A
    float gpa = 0.0f, vtg = 0.0f, va = 0.0f;
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      gpa = fmaf(GP[i * 16 + k], A[j * 16 + k], gpa);
      vtg = fmaf(V[k * 16 + i], GP[k * 16 + j], vtg);
      va = fmaf(V[i * 16 + k], A[k * 16 + j], va);
    }
    gv -= c * gpa;
    dAl -= c * vtg;
    dc -= GP[tid] * va;
  }
  W1[tid] = gv;
  __syncthreads();
  float xv = 0.0f;
#pragma unroll
  for (int k = 0; k < 16; ++k) xv = fmaf(V[k * 16 + i], W1[k * 16 + j], xv);  // V^T GV'
  W2[tid] = xv;
  __syncthreads();
  float dN = 0.0f;
#pragma unroll
  for (int k = 0; k < 16; ++k) dN = fmaf(W2[i * 16 + k], V[j * 16 + k], dN);  // (V^T GV') V^T
  dN = -dN;
  const bool pade = scheme == EWS_EXPM_PADE;
  const float alpha = scheme == EWS_EXPM_EULER ? c : 0.5f * c;
  const float dalpha = scheme == EWS_EXPM_EULER ? 1.0f : 0.5f;
  dAl = fmaf(alpha, dN, dAl);
  dc = fmaf(dN, dalpha * A[tid] + (pade ? c * (1.0f / 6.0f) * 2.0f * sp[2][tid] : 0.0f), dc);
  if (pade) {  // beta (dN A^T + A^T dN), beta = c^2 / 12
    __syncthreads();
    W1[tid] = dN;
    __syncthreads();
    float t2 = 0.0f;
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      t2 = fmaf(W1[i * 16 + k], A[j * 16 + k], t2);
      t2 = fmaf(A[k * 16 + i], W1[k * 16 + j], t2);
    }
    dAl = fmaf(c * c * (1.0f / 12.0f), t2, dAl);
  }
  return block_sum(dc, red, tid);
}

// Adjoint of the interval's flow M = expm_scheme(-hf A) (chen_expm) for the workgroup, given its cotangent G in LDS
// (overwritten); returns the cotangent of hf (zero for the identity flow). Scratch: Esq (SQMAX matrices), W1..W3
// (256, 256, 256 + 32 floats).
__device__ float block_flow_adjoint(const Args& a, const LdsTable* sp, float norm1, float hf, bool ident, float* G,
                                   float (*Esq)[256], float* W1, float* W2, float* W3, float* red, float* H,
                                   float& dAl, int tid) {
  if (ident) return 0.0f;
  if (a.chen_expm == EWS_EXPM_EXACT) return block_exp_adjoint(sp, norm1, hf, G, nullptr, Esq, Esq, red, H, tid);
  if (a.chen_expm == EWS_EXPM_EULER) {  // M = I - hf A
    dAl = fmaf(-hf, G[tid], dAl);
    return block_sum(-G[tid] * sp[1][tid], red, tid);
  }
  if (tid < 64) wave_matfn(sp, norm1, a.chen_expm, hf, false, W1, W2, W3, tid);  // V (and P, unused) of the step
  __syncthreads();
  return block_rational_adjoint(sp, a.chen_expm, hf, W2, G, nullptr, W1, W3, red, dAl, tid);
}

// Coefficient of a letter from its stage's base (series-leaf adjoint): b_{a+m} = c P_m b_a with
// c = (-h)^m / C(a + m, m) = prod_{j=1..m} (-h) j / (a + j); returns (c, dc/dh).
__device__ __forceinline__ float2 letter_coef(float h, int a, int m) {
  float k = 1.0f, hp = 1.0f;  // prod j / (a + j); (-h)^(m-1)
  for (int jj = 1; jj <= m; ++jj) {
    k *= (float)jj * frcp(a + jj);
    if (jj < m) hp *= -h;
  }
  return float2{-h * hp * k, -(float)m * hp * k};
}

template <int N, bool EXACTF>  // EXACTF: exact flows (the other schemes' code is left out)
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(EXACTF ? 3 : 1))) void k_leaf_bwd(Args a, LeafBwd o) {
  constexpr int LW = lw_of(N);
  __shared__ __align__(16) float sp[HP][256];
  // ds3 of the level adjoint and, after it, the flow adjoint's squarings / scratch share one region
  // 16 x 16 matrices and the rows of ds3 sit at a pitch of 17 floats (LP), so that a column read (16 lanes on
  // consecutive rows) and a row read (lanes on consecutive columns) both hit distinct banks
  constexpr int LP = 17;
  constexpr int UNF = (EXACTF ? SQMAX * 256 : 800) > (N >= 3 ? 256 * LP : 0) ? (EXACTF ? SQMAX * 256 : 800)
                                                                            : (N >= 3 ? 256 * LP : 0);
  __shared__ __align__(16) float UN[UNF];
  constexpr int TPT = QMAX + 4;  // row pitch of the transposed letters (QMAX + 1 columns)
  __shared__ __align__(16) float dS2[16 * LP], Gm[256];
  __shared__ __align__(16) float LtT[N >= 3 ? 16 * TPT : 1];
  __shared__ float2 s_lc[PM];  // the letter coefficients of a stage and their h-derivatives
  __shared__ float dS1[16], red[8];
  extern __shared__ __align__(16) float dyn[];  // the six letter arrays, (q + 1) x 16 each
  typedef float Row16[16];
  const int QN = a.q + 1;
  Row16* Lt = reinterpret_cast<Row16*>(dyn);
  Row16* G1 = Lt + QN;
  Row16* BT = G1 + QN;
  Row16* dB = BT + QN;
  Row16* dG1 = dB + QN;
  Row16* dBT = dG1 + QN;
  float* dS3 = UN;
  typedef float Mat[256];
  Mat* Esq = reinterpret_cast<Mat*>(UN);
  float *W1 = UN, *W2 = UN + 256, *W3 = UN + 512;
  const int tid = threadIdx.x, i = tid >> 4, j = tid & 15;
  const int q = a.q;
  stage_lds(&sp[0][0], a.apow, HP * 256, tid, 256);
  const float norm1 = a.apow[a.npow * 256];
  float H[HP];
#pragma unroll
  for (int p = 0; p < HP; ++p) H[p] = 0.0f;
  float dAl = 0.0f;
  const int l = tid & 63;
  __syncthreads();
  const long total = (long)a.B * a.n_int;
  // depth 3: the next interval's inputs (ds3 as four float4 per thread, ds2, dM, ds1 and the increment) are loaded
  // into registers once the degree loop is done, so that their latency hides behind the rest of the interval
  f4 pf3[4];
  float pf2 = 0.0f, pfg = 0.0f, pfs1 = 0.0f, pfv = 0.0f, pft0 = 0.0f, pft1 = 0.0f;
  auto prefetch = [&](long it2) {
    const int b2 = (int)(it2 / a.n_int), t2 = (int)(it2 - (long)b2 * a.n_int);
    const float* dr = a.loc + ((size_t)b2 * a.n_int + t2) * LW;
    const float* th2 = a.clock + (size_t)b2 * a.L + t2;  // the clock values around the interval
    pft0 = th2[0];
    pft1 = th2[1];
#pragma unroll
    for (int m = 0; m < 4; ++m) pf3[m] = *reinterpret_cast<const f4*>(dr + 272 + 4 * tid + 1024 * m);
    pf2 = dr[16 + tid];
    pfg = a.fl[((size_t)b2 * a.n_int + t2) * 256 + tid];
    if (tid < 16) {
      const float* x = a.path + ((size_t)b2 * a.L + t2) * a.d;
      pfv = tid < a.d ? x[a.d + tid] - x[tid] : 0.0f;
      pfs1 = dr[tid];
    }
  };
  if constexpr (N >= 3) {
    if (blockIdx.x < total) prefetch(blockIdx.x);
  }
  const int tid_all = tid;
  for (long it = blockIdx.x; it < total; it += gridDim.x) {
    // lane indices from an opaque copy of the thread index: the interval's addresses are recomputed, not held live
    const int tid = opaque_vgpr(tid_all), i = tid >> 4, j = tid & 15, l = tid & 63;
    const int b = (int)(it / a.n_int), t = (int)(it - (long)b * a.n_int);
    const float* th = a.clock + (size_t)b * a.L;
    const float h = N >= 3 ? pft1 - pft0 : th[t + 1] - th[t];  // depth 3: from the registers
    const float* drow = a.loc + ((size_t)b * a.n_int + t) * LW;  // ds_t
    // ---- inputs
    if constexpr (N >= 3) {  // from the registers; ds3[a][b][c] at (16 a + b) LP + c
      if (tid < 16) {
        Lt[0][tid] = pfv;
        dS1[tid] = pfs1;
      }
      dS2[i * LP + j] = pf2;
#pragma unroll
      for (int m = 0; m < 4; ++m) {
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const int e = 4 * tid + 1024 * m + c;
          dS3[(e >> 4) * LP + (e & 15)] = pf3[m][c];
        }
      }
      Gm[tid] = pfg;
    } else {
      if (tid < 16) {
        const float* x = a.path + ((size_t)b * a.L + t) * a.d;
        const float v = tid < a.d ? x[a.d + tid] - x[tid] : 0.0f;
        Lt[0][tid] = v;
        dS1[tid] = drow[tid];
      }
      if constexpr (N >= 2) dS2[i * LP + j] = drow[16 + tid];
      Gm[tid] = a.fl[((size_t)b * a.n_int + t) * 256 + tid];  // dM_t
    }
    for (int e = tid; e < QN * 16; e += 256) {
      (&dB[0][0])[e] = 0.0f;
      (&dBT[0][0])[e] = 0.0f;
    }
    __syncthreads();
    // ---- letters b_p = (-h)^p A^p v / p!, by stages from the powers table P_m = A^m / m!: the letters a + m of
    // the stage on base letter a (a = 0, PM, 2 PM, ...; m = 1 .. PM) are b_{a+m} = c_{a,m} P_m b_a with
    // c_{a,m} = (-h)^m / C(a + m, m), all of a stage at once (thread: power m, row r)
    for (int a0 = 0; a0 < q; a0 += PM) {
      if (tid < PM) s_lc[tid] = letter_coef(h, a0, tid + 1);
      __syncthreads();
      for (int e = tid; e < PM * 16; e += 256) {
        const int m = 1 + (e >> 4), r = e & 15, p = a0 + m;
        if (p <= q) {
          float x = 0.0f;
#pragma unroll 4
          for (int k = 0; k < 16; ++k) {
            const int kk = (k + r) & 15;  // rotated so that the 16 rows of a power hit distinct banks
            x = fmaf(sp[m][r * 16 + kk], Lt[a0][kk], x);
          }
          Lt[p][r] = s_lc[m - 1].x * x;
        }
      }
      __syncthreads();
    }
    for (int e = tid; e < (q + 1) * 16; e += 256) {
      const int n = e >> 4, r = e & 15;
      G1[n][r] = Lt[n][r] * frcp(n + 1);
      dG1[n][r] = dS1[r];
    }
    if constexpr (N >= 2) {
      for (int e = tid; e < (q + 1) * 16; e += 256) {
        const int n = e >> 4, r = e & 15;
        float sacc = 0.0f;
        for (int p = 0; p + n <= q; ++p) sacc = fmaf(Lt[p][r], frcp(p + n + N), sacc);
        BT[n][r] = sacc;
      }
    }
    __syncthreads();
    // ---- level adjoints
    if constexpr (N == 2) {
      // dbt2_n = ds2 g1_n;  dg1_n += ds2^T bt2_n
      for (int e = tid; e < (q + 1) * 16; e += 256) {
        const int n = e >> 4, r = e & 15;
        float x1 = 0.0f, x2 = 0.0f;
#pragma unroll
        for (int k = 0; k < 16; ++k) {
          x1 = fmaf(dS2[r * LP + k], G1[n][k], x1);
          x2 = fmaf(dS2[k * LP + r], BT[n][k], x2);
        }
        dBT[n][r] = x1;
        dG1[n][r] += x2;
      }
      __syncthreads();
    }
    if constexpr (N == 3) {
      // per degree NN: dg2_NN = bt3_NN ._1 ds3 + ds2 (F) and E_NN = ds3 ._3 g1_NN (F2), then
      //   pairs (p, n = NN - p): db_p += dg2_NN g1_n / (NN+2);  dg1_n += dg2_NN^T b_p / (NN+2)
      //   dbt3_{p+NN} += (E_NN b_p) / (p+NN+2)
      // The three pair sums are products of a 16 x 16 matrix with up to QMAX + 1 letter columns, accumulated over
      // NN on fp32 MFMA: wavefront 0 holds db (columns p), wavefront 1 dg1 (columns n), wavefront 2 dbt3 (columns
      // s = p + NN, its 1 / (s + 2) applied at the end); the B operands read the letters transposed (LtT; g1_n =
      // b_n / (n + 1)) so that the 16 lanes of a k-step read 16 consecutive columns.
      for (int e = tid; e < 16 * QN; e += 256) {
        const int n = e >> 4, r = e & 15;
        LtT[r * TPT + n] = Lt[n][r];
      }
      __syncthreads();  // LtT
      // Each of the three wavefronts forms the A operand of its own pair sum for every degree in registers, from
      // the lane's 64 entries of ds3 read once (no LDS round trip and no barrier per degree):
      //   wavefront 0: F[li][k] = ds2[li][k] + sum_c bt3_NN[c] ds3[c][li][k]   (k = 4 ks + lk)
      //   wavefront 1: F[k][li] = ds2[k][li] + sum_c bt3_NN[c] ds3[c][k][li]
      //   wavefront 2: E[li][k] = sum_c ds3[li][k][c] g1_NN[c]
      const int wv = tid >> 6, li = l & 15, lk = l >> 4;
      f4 acc[3];
#pragma unroll
      for (int tt = 0; tt < 3; ++tt) acc[tt] = f4{0.0f, 0.0f, 0.0f, 0.0f};
      const int ntile = (QN + 15) >> 4;  // column tiles of 16 (QN <= QMAX + 1 = 41: at most 3)
      if (wv < 3) {
        float d3[4][16], d2[4];
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
          const int k = 4 * ks + lk;
#pragma unroll
          for (int c = 0; c < 16; ++c)
            d3[ks][c] = wv == 0 ? dS3[(16 * c + li) * LP + k] : wv == 1 ? dS3[(16 * c + k) * LP + li]
                                                                       : dS3[(16 * li + k) * LP + c];
          d2[ks] = wv == 0 ? dS2[li * LP + k] : wv == 1 ? dS2[k * LP + li] : 0.0f;
        }
        for (int NN = 0; NN <= q; ++NN) {
          const float* vrow = wv == 2 ? G1[NN] : BT[NN];  // the same row for every lane
          const float inv2 = wv == 2 ? 1.0f : frcp(NN + 2);
          float av[4];
#pragma unroll
          for (int ks = 0; ks < 4; ++ks) {
            float x = d2[ks];
#pragma unroll
            for (int c = 0; c < 16; ++c) x = fmaf(vrow[c], d3[ks][c], x);
            av[ks] = inv2 * x;  // A[row li][k = 4 ks + lk]
          }
#pragma unroll
          for (int tt = 0; tt < 3; ++tt) {
            // a tile of columns 16 tt .. 16 tt + 15 holds a valid letter index only if 16 tt <= NN (db, dg1: NN - col
            // >= 0) or 16 tt + 15 >= NN (dbt3: col - NN >= 0); the others add exact zeros and are skipped
            if (tt < ntile && (wv == 2 ? 16 * tt + 15 >= NN : 16 * tt <= NN)) {
              const int col = 16 * tt + li;  // p (db), n (dg1) or s (dbt3)
              // letter index of column col: NN - col (db: g1, dg1: b) or col - NN (dbt3: b), zero outside [0, q]
              const int src = wv == 2 ? col - NN : NN - col;
              const bool ok = src >= 0 && src <= q && col <= q;
              const int sv = ok ? src : 0;
              const float gs = ok ? (wv == 0 ? frcp(sv + 1) : 1.0f) : 0.0f;
#pragma unroll
              for (int ks = 0; ks < 4; ++ks) acc[tt] = mfma(av[ks], gs * LtT[(4 * ks + lk) * TPT + sv], acc[tt]);
            }
          }
        }
      }
      // accumulators: lane l holds rows 4 (l / 16) + r of column 16 tt + l % 16
      if (wv < 3) {
#pragma unroll
        for (int tt = 0; tt < 3; ++tt) {
          const int col = 16 * tt + li;
          if (tt < ntile && col <= q) {
            const float sc = wv == 2 ? frcp(col + 2) : 1.0f;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              const int row = 4 * lk + r;
              if (wv == 0) dB[col][row] += acc[tt][r];
              else if (wv == 1) dG1[col][row] += acc[tt][r];
              else dBT[col][row] += sc * acc[tt][r];
            }
          }
        }
      }
      if (it + gridDim.x < total) prefetch(it + gridDim.x);
      __syncthreads();
    }
    // bt_N -> b_p; g1_n -> b_n
    for (int e = tid; e < (q + 1) * 16; e += 256) {
      const int p = e >> 4, r = e & 15;
      float x = fmaf(dG1[p][r], frcp(p + 1), dB[p][r]);
      if constexpr (N >= 2) {
        for (int NN = 0; NN + p <= q; ++NN) x = fmaf(dBT[NN][r], frcp(p + NN + N), x);
      }
      dB[p][r] = x;
    }
    __syncthreads();
    // ---- the letters in reverse, stage by stage (the last first): for p = a + m, z_p = P_m^T db_p,
    // db_a += c_{a,m} z_p, dh += (d c_{a,m} / dh) <z_p, b_a>, and the cotangent of A^m gains
    // (c_{a,m} / m!) db_p (x) b_a (H_m, turned into dA once per launch with the flows' terms)
    float dhl = 0.0f;  // partial dh in threads 0 .. 15
    Row16* Zt = dBT;   // free after the degree sums
    for (int a0 = q > 0 ? ((q - 1) / PM) * PM : -1; a0 >= 0; a0 -= PM) {
      if (tid < PM) s_lc[tid] = letter_coef(h, a0, tid + 1);
      for (int e = tid; e < PM * 16; e += 256) {
        const int m = 1 + (e >> 4), jj = e & 15, p = a0 + m;
        float z = 0.0f;
        if (p <= q) {
#pragma unroll
          for (int i2 = 0; i2 < 16; ++i2) z = fmaf(sp[m][i2 * 16 + jj], dB[p][i2], z);
        }
        Zt[m - 1][jj] = z;
      }
      __syncthreads();  // the stage's coefficients and z
      {
        const float bj = Lt[a0][j];
        float ifact = 1.0f;
#pragma unroll
        for (int m = 1; m <= PM; ++m) {
          ifact *= 1.0f / (float)m;
          const int p = a0 + m;
          if (p <= q) H[m] = fmaf(s_lc[m - 1].x * ifact * dB[p][i], bj, H[m]);
        }
      }
      if (tid < 16) {
        float acc = dB[a0][tid], dz = 0.0f;
        for (int m = 1; m <= PM && a0 + m <= q; ++m) {
          const float2 cc = s_lc[m - 1];
          const float z = Zt[m - 1][tid];
          acc = fmaf(cc.x, z, acc);
          dz = fmaf(cc.y, z, dz);
        }
        dB[a0][tid] = acc;
        dhl = fmaf(dz, Lt[a0][tid], dhl);
      }
      __syncthreads();
    }
    // ---- flow adjoint
    bool ident = false;
    const float hf = a.flow_mode == EWS_FLOW_PER_INTERVAL ? h : flow_step(a, th, t, ident);
    const float dhf = EXACTF ? (ident ? 0.0f : block_exp_adjoint(sp, norm1, hf, Gm, nullptr, Esq, Esq, red, H, tid))
                             : block_flow_adjoint(a, sp, norm1, hf, ident, Gm, Esq, W1, W2, W3, red, H, dAl, tid);
    // ---- outputs
    if (tid < 16) o.dv[((size_t)b * a.n_int + t) * 16 + tid] = dB[0][tid];
    {
      float v = dhl;  // nonzero in lanes 0 .. 15 of wavefront 0
      v = lanes::sum16(v);
      if (tid == 0) red[4] = v;
    }
    __syncthreads();
    if (tid == 0) {
      const float dl = red[4];
      if (a.flow_mode == EWS_FLOW_PER_INTERVAL) {
        o.dh[(size_t)b * a.n_int + t] = dl + dhf;
      } else {
        o.dh[(size_t)b * a.n_int + t] = dl;
      }
      // the shared step's cotangent per interval, summed in a fixed order by k_dsh_reduce
      o.dshi[2 * ((size_t)b * a.n_int + t)] = (a.flow_mode != EWS_FLOW_PER_INTERVAL && !ident) ? dhf : 0.0f;
      o.dshi[2 * ((size_t)b * a.n_int + t) + 1] = 0.0f;
    }
    __syncthreads();
  }
  float* pb = o.part + (size_t)blockIdx.x * (HP + 1) * 256;
#pragma unroll
  for (int p = 0; p < HP; ++p) pb[p * 256 + tid] = H[p];
  pb[HP * 256 + tid] = dAl;
}

// Van Loan leaf adjoint (one workgroup per interval, grid-stride). The forward's recompute saved per interval the
// step matrices P, V and the knot increments Delta_m (Delta_{M-1} = V w, Delta_{m-1} = P Delta_m); from them
// Pre_m, R_m, Y_m, X_m (see k_vl), then:
//   level adjoints:  dDelta_m += dS1;  dY_m = dS2 Delta_m, dDelta_m += dS2^T Y_m;
//     depth 3 (S3 = sum_m Delta_m[b] G_m[a][c], G_m = Y_m (x) R_m + X_m (x) Delta_m / 2), with
//     Q_m = dS3 ._2 Delta_m:  dY_m += Q_m R_m,  dX_m = Q_m Delta_m / 2,  dR_m = Q_m^T Y_m,
//     dDelta_m += Q_m^T X_m / 2 (last index) and dDelta_m[b] += <dS3[:, b, :], G_m> (middle index);
//     each thread keeps its column dS3[a][:][c] and its row dS3[a][b][:] in registers across the segments;
//   Y = Pre + Delta/2, X = Pre + Delta/3, Pre_m = sum_{j<m} Delta_j, R_m = sum_{j>m} Delta_j;
//   chain (one wavefront): lambda_0 = dDelta_0, lambda_m = dDelta_m + P^T lambda_{m-1},
//   GP = sum_m lambda_{m-1} (x) Delta_m, GV = lambda_{M-1} (x) w, dw = V^T lambda_{M-1}, dv = dw / M;
//   step matrices: block_exp_adjoint (exact) or block_rational_adjoint, for the step delta = h / M.
// Then the flow's adjoint as in k_leaf_bwd.
constexpr int VMAX = 64;  // knots per interval at most

template <int N, bool EXACTF>
__global__ __launch_bounds__(256) void k_vl_bwd(Args a, LeafBwd o) {
  constexpr int LW = lw_of(N);
  __shared__ __align__(16) float sp[HP][256];
  __shared__ __align__(16) float Pm[256], Vm[256], W1[256], W2[256], W3[256 + 32], GPm[256], GVm[256], Gm[256];
  // The knot arrays and dS3 are dead once the chain has run; the squarings of the step-matrix and flow adjoints
  // (Esq, Fsq) then reuse their space, which keeps the workgroup at two per CU.
  constexpr int UL = 7 * VMAX * 16 + (N >= 3 ? 4096 : 4), UE = 2 * SQMAX * 256;
  __shared__ __align__(16) float U[UL > UE ? UL : UE];
  __shared__ __align__(16) float dS2[256];
  typedef float Row16[16];
  typedef float Mat[256];
  Row16* Dl = reinterpret_cast<Row16*>(U);
  Row16* Rs = Dl + VMAX;
  Row16* Ys = Rs + VMAX;
  Row16* Xs = Ys + VMAX;
  Row16* dD = Xs + VMAX;
  Row16* dP = dD + VMAX;
  Row16* dR = dP + VMAX;
  float* dS3 = U + 7 * VMAX * 16;
  Mat* Esq = reinterpret_cast<Mat*>(U);
  Mat* Fsq = Esq + SQMAX;
  __shared__ __align__(16) float dS1[16], wv[16], lam[16], red[8];
  // depth 3: per-wavefront partial sums of the column cotangents of a block of VB knots, summed in a fixed order
  // once per block
  constexpr int VB = 8;
  __shared__ float wR[VB][4][16], wD[VB][4][16], rowD[VB][16];
  const int tid = threadIdx.x, i = tid >> 4, j = tid & 15, l = tid & 63, g = l >> 4, c16 = l & 15;
  const int wv_id = tid >> 6;
  const int Mv = a.vm, vs = 512 + 16 * Mv;
#pragma unroll
  for (int p = 0; p < HP; ++p) sp[p][tid] = a.apow[p * 256 + tid];
  const float norm1 = a.apow[a.npow * 256];
  float H[HP];
#pragma unroll
  for (int p = 0; p < HP; ++p) H[p] = 0.0f;
  float dAl = 0.0f;
  __syncthreads();
  const long total = (long)a.B * a.n_int;
  // ---- saved step matrices and increments, loaded into registers during the interval before (issued once the
  // depth-3 sums are done): P, V, the knots (one float4 per thread: M <= 64), ds1, ds2, ds3 (four float4), dM and the
  // increment's coordinates; all of them before the first store to LDS
  const bool dl_own = tid < Mv * 4;
  float in_p = 0.0f, in_v = 0.0f, in_g = 0.0f, in_s2 = 0.0f, in_s1 = 0.0f, in_x0 = 0.0f, in_x1 = 0.0f;
  f4 in_d = {0.0f, 0.0f, 0.0f, 0.0f};
  f4 in_s3[N >= 3 ? 4 : 1];
  auto prefetch = [&](long i2) {
    const size_t r2 = (size_t)i2;  // = b2 n_int + t2
    const int b2 = (int)(i2 / a.n_int), t2 = (int)(i2 - (long)b2 * a.n_int);
    const float* sv2 = a.vlsave + r2 * vs;
    const float* dr2 = a.loc + r2 * LW;
    in_p = sv2[tid];
    in_v = sv2[256 + tid];
    in_g = a.fl[r2 * 256 + tid];  // dM_t
    if (dl_own) in_d = reinterpret_cast<const f4*>(sv2 + 512)[tid];
    if constexpr (N >= 2) in_s2 = dr2[16 + tid];
    if constexpr (N >= 3) {
#pragma unroll
      for (int m = 0; m < 4; ++m) in_s3[m] = reinterpret_cast<const f4*>(dr2 + 272)[tid + 256 * m];
    }
    if (tid < 16) {
      in_s1 = dr2[tid];
      if (tid < a.d) {
        const float* x = a.path + ((size_t)b2 * a.L + t2) * a.d;
        in_x0 = x[tid];
        in_x1 = x[a.d + tid];
      }
    }
  };
  if (blockIdx.x < total) prefetch(blockIdx.x);
  for (long it = blockIdx.x; it < total; it += gridDim.x) {
    const int b = (int)(it / a.n_int), t = (int)(it - (long)b * a.n_int);
    const float* th = a.clock + (size_t)b * a.L;
    const float in_w = (tid < 16 && tid < a.d) ? (in_x1 - in_x0) / (float)Mv : 0.0f;
    bool fixed = false;  // delta = 0: P = V = I (the jump / basepoint interval), no dependence on A or the clock
    float delta;
    if (a.vl_mode == EWS_FLOW_PER_INTERVAL) {
      delta = (th[t + 1] - th[t]) / (float)Mv;
    } else {
      delta = vl_shared_step(a, th);
      fixed = delta == 0.0f || (a.vl_mode == EWS_FLOW_CACHED_BASEPOINT && t == 0);
    }
    Pm[tid] = in_p;
    Vm[tid] = in_v;
    if (dl_own) reinterpret_cast<f4*>(U)[tid] = in_d;  // Dl[m][c] at U[16 m + c]
    if (tid < 16) {
      wv[tid] = in_w;
      dS1[tid] = in_s1;
    }
    if constexpr (N >= 2) dS2[tid] = in_s2;
    if constexpr (N >= 3) {
#pragma unroll
      for (int m = 0; m < 4; ++m) reinterpret_cast<f4*>(dS3)[tid + 256 * m] = in_s3[m];
    }
    Gm[tid] = in_g;
    __syncthreads();
    {  // Pre, R, Y, X; level-1 cotangent; zero the other accumulators. 16 lanes per column, a segment of
       // ceil(M / 16) knots each: the segments' sums scanned across the lanes, then each lane walks its segment
      const int col = tid >> 4, seg = tid & 15, S = (Mv + 15) >> 4, m0 = min(Mv, seg * S), m1 = min(Mv, m0 + S);
      float own = 0.0f;
      for (int m = m0; m < m1; ++m) own += Dl[m][col];
      float inc = own;
#pragma unroll
      for (int o = 1; o < 16; o <<= 1) {
        const float v = __shfl_up(inc, o, 16);
        if (seg >= o) inc += v;
      }
      const float total = __shfl(inc, 15, 16);
      float pre = inc - own, suf = total - inc;
      for (int m = m0; m < m1; ++m) {
        const float dm = Dl[m][col];
        Ys[m][col] = fmaf(0.5f, dm, pre);
        Xs[m][col] = fmaf(1.0f / 3.0f, dm, pre);
        pre += dm;
        dD[m][col] = dS1[col];
        dP[m][col] = 0.0f;
        dR[m][col] = 0.0f;
      }
      for (int m = m1 - 1; m >= m0; --m) {  // R_m: the knots after m
        Rs[m][col] = suf;
        suf += Dl[m][col];
      }
    }
    __syncthreads();
    // ---- level adjoints
    if constexpr (N >= 2) {
      for (int e = tid; e < Mv * 16; e += 256) {  // dY_m = dS2 Delta_m;  dDelta_m += dS2^T Y_m
        const int m = e >> 4, r = e & 15;
        float y1 = 0.0f, y2 = 0.0f;
#pragma unroll
        for (int k = 0; k < 16; ++k) {
          y1 = fmaf(dS2[r * 16 + k], Dl[m][k], y1);
          y2 = fmaf(dS2[k * 16 + r], Ys[m][k], y2);
        }
        dP[m][r] += y1;
        dD[m][r] += fmaf(0.5f, y1, y2);
      }
      __syncthreads();
    }
    if constexpr (N >= 3) {
      float colb[16];  // dS3[i][.][j]
      f4 rowc[4];      // dS3[i][j][.]
#pragma unroll
      for (int k = 0; k < 16; ++k) colb[k] = dS3[i * 256 + k * 16 + j];
#pragma unroll
      for (int k = 0; k < 4; ++k) rowc[k] = *reinterpret_cast<const f4*>(dS3 + i * 256 + j * 16 + 4 * k);
      for (int mb = 0; mb < Mv; mb += VB) {
      const int me = min(Mv, mb + VB);
      for (int m = mb; m < me; ++m) {
        // the knot's Delta_m and R_m: the same 16 floats in every lane (broadcast float4 reads)
        float q = 0.0f, e1 = 0.0f, f1 = 0.0f;
#pragma unroll
        for (int k4 = 0; k4 < 4; ++k4) {
          const f4 dk = *reinterpret_cast<const f4*>(&Dl[m][4 * k4]);
          const f4 rk = *reinterpret_cast<const f4*>(&Rs[m][4 * k4]);
#pragma unroll
          for (int c = 0; c < 4; ++c) {
            q = fmaf(colb[4 * k4 + c], dk[c], q);
            e1 = fmaf(rowc[k4][c], rk[c], e1);
            f1 = fmaf(rowc[k4][c], dk[c], f1);
          }
        }
        const float yi = Ys[m][i], xi = Xs[m][i];
        // over the last index (lanes j of a row i): dY_m[i], dX_m[i]
        float py = q * Rs[m][j], px = 0.5f * q * Dl[m][j];
        py = lanes::sum16(py);
        px = lanes::sum16(px);
        // over the first index (rows i of the wave, then the four wavefronts' partials in a fixed order):
        // dR_m[j], dDelta_m[j]
        float pr2 = q * yi, pd = fmaf(0.5f * q, xi, fmaf(yi, e1, 0.5f * xi * f1));
        pr2 = lanes::add_xor32(lanes::add_xor16(pr2));
        pd = lanes::add_xor32(lanes::add_xor16(pd));
        const int sb = m - mb;
        if (j == 0) {  // row i lives in one wavefront: a single writer
          dP[m][i] += py + px;
          rowD[sb][i] = fmaf(0.5f, py, px * (1.0f / 3.0f));
        }
        if (l < 16) {
          wR[sb][wv_id][j] = pr2;
          wD[sb][wv_id][j] = pd;
        }
      }
      __syncthreads();
      {  // the block's partials: thread (knot mb + tid / 16, column tid % 16)
        const int sb = tid >> 4, c = tid & 15;
        if (sb < me - mb) {
          const int m = mb + sb;
          dR[m][c] += ((wR[sb][0][c] + wR[sb][1][c]) + wR[sb][2][c]) + wR[sb][3][c];
          dD[m][c] += rowD[sb][c] + (((wD[sb][0][c] + wD[sb][1][c]) + wD[sb][2][c]) + wD[sb][3][c]);
        }
      }
      __syncthreads();  // before the next block's partials
      }
    }
    if (it + gridDim.x < total) prefetch(it + gridDim.x);  // the next interval's inputs
    // Pre and R -> Delta (dP holds dPre): dDelta_m += sum_{m' > m} dPre_m' + sum_{m' < m} dR_m', segments as above
    {
      const int col = tid >> 4, seg = tid & 15, S = (Mv + 15) >> 4, m0 = min(Mv, seg * S), m1 = min(Mv, m0 + S);
      float ownP = 0.0f, ownR = 0.0f;
      for (int m = m0; m < m1; ++m) {
        ownP += dP[m][col];
        ownR += dR[m][col];
      }
      float incP = ownP, incR = ownR;
#pragma unroll
      for (int o = 1; o < 16; o <<= 1) {
        const float vp = __shfl_up(incP, o, 16), vr = __shfl_up(incR, o, 16);
        if (seg >= o) {
          incP += vp;
          incR += vr;
        }
      }
      float accP = __shfl(incP, 15, 16) - incP, accR = incR - ownR;
      for (int m = m1 - 1; m >= m0; --m) {
        dD[m][col] += accP;
        accP += dP[m][col];
      }
      for (int m = m0; m < m1; ++m) {
        dD[m][col] += accR;
        accR += dR[m][col];
      }
      if (seg == 0) lam[col] = dD[0][col];
    }
    __syncthreads();
    // ---- the chain in reverse, one wavefront
    if (tid < 64) {
      f4 pc;  // P[4g + r][c16]
#pragma unroll
      for (int r = 0; r < 4; ++r) pc[r] = Pm[(4 * g + r) * 16 + c16];
      const int gi = l >> 2, gj = 4 * (l & 3);
      f4 gp = {0.0f, 0.0f, 0.0f, 0.0f};
      for (int m = 1; m < Mv; ++m) {
        const f4 lv = *reinterpret_cast<const f4*>(lam + 4 * g);
        const float li = lam[gi];
        const f4 dm = *reinterpret_cast<const f4*>(&Dl[m][gj]);
#pragma unroll
        for (int r = 0; r < 4; ++r) gp[r] = fmaf(li, dm[r], gp[r]);
        float u = fmaf(pc.x, lv.x, fmaf(pc.y, lv.y, fmaf(pc.z, lv.z, pc.w * lv.w)));
        u = lanes::add_xor32(lanes::add_xor16(u));
        wave_order_d();
        if (g == 0) lam[c16] = dD[m][c16] + u;
        wave_order_d();
      }
      *reinterpret_cast<f4*>(GPm + 4 * l) = gp;
    }
    __syncthreads();
    GVm[tid] = lam[i] * wv[j];
    {
      float u = Vm[j * 16 + i] * lam[j];  // (V^T lambda)[i]
      u = lanes::sum16(u);
      if (j == 0) o.dv[((size_t)b * a.n_int + t) * 16 + i] = u / (float)Mv;
    }
    __syncthreads();
    // ---- step matrices' adjoint
    float ddelta = 0.0f;
    if (!fixed) {
      if (a.vl_expm == EWS_EXPM_EXACT)
        ddelta = block_exp_adjoint(sp, norm1, delta, GPm, GVm, Esq, Fsq, red, H, tid);
      else
        ddelta = block_rational_adjoint(sp, a.vl_expm, delta, Vm, GPm, GVm, W1, W2, red, dAl, tid);
    }
    // ---- flow adjoint
    bool ident;
    const float hf = flow_step(a, th, t, ident);
    const float dhf = EXACTF ? (ident ? 0.0f : block_exp_adjoint(sp, norm1, hf, Gm, nullptr, Esq, Esq, red, H, tid))
                             : block_flow_adjoint(a, sp, norm1, hf, ident, Gm, Esq, W1, W2, W3, red, H, dAl, tid);
    if (tid == 0) {
      float dh = 0.0f, s_flow = 0.0f, s_vl = 0.0f;  // shared steps: summed in a fixed order by k_dsh_reduce
      if (a.vl_mode == EWS_FLOW_PER_INTERVAL) dh += ddelta / (float)Mv;
      else if (!fixed) s_vl = ddelta / (float)Mv;
      if (a.flow_mode == EWS_FLOW_PER_INTERVAL) dh += dhf;
      else if (!ident) s_flow = dhf;
      o.dh[(size_t)b * a.n_int + t] = dh;
      o.dshi[2 * ((size_t)b * a.n_int + t)] = s_flow;
      o.dshi[2 * ((size_t)b * a.n_int + t) + 1] = s_vl;
    }
    __syncthreads();
  }
  float* pb = o.part + (size_t)blockIdx.x * (HP + 1) * 256;
#pragma unroll
  for (int p = 0; p < HP; ++p) pb[p * 256 + tid] = H[p];
  pb[HP * 256 + tid] = dAl;
}

// sums of the workgroups' partials (float64): workgroup (p, c) sums row p of the partial sets c, c + PRS, ...
constexpr int PRS = 32;  // partial-sum slices (the second level of the reduction is in k_dA)
__global__ __launch_bounds__(256) void k_part_reduce(const float* part, int nparts, double* hsum) {
  const int p = blockIdx.x, c = blockIdx.y, tid = threadIdx.x;
  double s0 = 0.0, s1 = 0.0;
  int k = c;
  for (; k + PRS < nparts; k += 2 * PRS) {
    s0 += (double)part[((size_t)k * (HP + 1) + p) * 256 + tid];
    s1 += (double)part[((size_t)(k + PRS) * (HP + 1) + p) * 256 + tid];
  }
  if (k < nparts) s0 += (double)part[((size_t)k * (HP + 1) + p) * 256 + tid];
  hsum[((size_t)c * (HP + 1) + p) * 256 + tid] = s0 + s1;
}

// dA = sum_p sum_{j<p} (A^T)^j H_p (A^T)^{p-1-j} + the direct terms (float64):
// R_{P-1} = H_P, R_j = H_{j+1} + R_{j+1} A^T, dA = R_0 + A^T (R_1 + A^T (R_2 + ...)), P = PM.
__global__ __launch_bounds__(256) void k_dA(Args a, const double* hsum, float* grad_A) {
  __shared__ double At[256], Rs[PM][256], U[256], Hs[HP + 1][256];
  const int tid = threadIdx.x, i = tid >> 4, j = tid & 15;
  for (int p = 0; p <= HP; ++p) {
    double v = 0.0;
    for (int c = 0; c < PRS; ++c) v += hsum[((size_t)c * (HP + 1) + p) * 256 + tid];
    Hs[p][tid] = v;
  }
  At[tid] = (double)a.apow[256 + j * 16 + i];  // A^T[i][j]
  Rs[PM - 1][tid] = Hs[PM][tid];
  __syncthreads();
  for (int jj = PM - 2; jj >= 0; --jj) {
    double v = Hs[jj + 1][tid];
    for (int k = 0; k < 16; ++k) v += Rs[jj + 1][i * 16 + k] * At[k * 16 + j];
    Rs[jj][tid] = v;
    __syncthreads();
  }
  U[tid] = Rs[PM - 1][tid];
  __syncthreads();
  for (int jj = PM - 2; jj >= 0; --jj) {
    double v = Rs[jj][tid];
    for (int k = 0; k < 16; ++k) v += At[i * 16 + k] * U[k * 16 + j];
    __syncthreads();
    U[tid] = v;
    __syncthreads();
  }
  if (i < a.d && j < a.d) grad_A[i * a.d + j] = (float)(U[tid] + Hs[HP][tid]);
}

// dsh[b] = sum over the intervals of dshi[b] (both slots), a workgroup per sample: strided partials, then a fixed
// tree, so the sum does not depend on scheduling
__global__ __launch_bounds__(256) void k_dsh_reduce(Args a, LeafBwd o) {
  __shared__ float r0[256], r1[256];
  const int b = blockIdx.x, tid = threadIdx.x;
  const float* src = o.dshi + (size_t)b * a.n_int * 2;
  float s0 = 0.0f, s1 = 0.0f;
  for (int t = tid; t < a.n_int; t += 256) {
    s0 += src[2 * t];
    s1 += src[2 * t + 1];
  }
  r0[tid] = s0;
  r1[tid] = s1;
  __syncthreads();
  for (int w = 128; w > 0; w >>= 1) {
    if (tid < w) {
      r0[tid] += r0[tid + w];
      r1[tid] += r1[tid + w];
    }
    __syncthreads();
  }
  if (tid == 0) {
    o.dsh[2 * b] = r0[0];
    o.dsh[2 * b + 1] = r1[0];
  }
}

// ------------------------------------------------------------------------------------------------ block-series level 1
// Level 1 of the block-series leaf (ews/core/kernels/blockdiag_engine.py:81-136, ews/core/leaf.py:138-175): the
// reference reads G = phi(X) = int_0^1 e^{sX} ds, X = -h A, off one augmented exponential per interval,
// exp([[X, I], [0, 0]]) = [[e^X, phi(X)], [0, I]], and writes s1 = G v at any step; its level 2 is the series
// leaf's (k_local at the order q, which runs first; this kernel overwrites its level 1). Here phi and e^X come from
// the powers table (P_p = A^p / p!): on Y = X / 2^s with ||Y||_1 <= 1, phi(Y) = sum_p y^p P_p / (p + 1) and
// e^Y = sum_p y^p P_p (degree PM, y = -h / 2^s: remainder below 1/14!), then s doublings
// phi(2Y) = phi(Y) (e^Y + I) / 2, e^{2Y} = (e^Y)^2. One workgroup of 256 threads per interval (grid-stride), thread
// (i, j) one entry of the 16 x 16 (padded) matrices.
__device__ __forceinline__ float inv_int(int n) { return 1.0f / (float)n; }

__global__ __launch_bounds__(256) void k_bs_level1(Args a) {
  __shared__ float sp[PM + 1][256];
  __shared__ float gm[256], em[256];
  __shared__ float vv[16];
  const int tid = threadIdx.x, i = tid >> 4, j = tid & 15;
  stage_lds(&sp[0][0], a.apow, (PM + 1) * 256, tid, 256);
  const float norm1 = a.apow[a.npow * 256];
  __syncthreads();
  const long total = (long)a.B * a.n_int;
  for (long it = blockIdx.x; it < total; it += gridDim.x) {
    const int b = (int)(it / a.n_int), t = (int)(it - (long)b * a.n_int);
    const float* th = a.clock + (size_t)b * a.L;
    const float h = th[t + 1] - th[t];
    if (tid < 16) {
      const float* x = a.path + ((size_t)b * a.L + t) * a.d;
      vv[tid] = tid < a.d ? x[a.d + tid] - x[tid] : 0.0f;
    }
    int s = 0;
    float xn = fabsf(h) * norm1;
    while (xn > 1.0f && s < SQMAX) {
      xn *= 0.5f;
      ++s;
    }
    const float y = -h * ldexpf(1.0f, -s);
    float g = sp[PM][tid] * inv_int(PM + 1), e = sp[PM][tid];
#pragma unroll
    for (int p = PM - 1; p >= 0; --p) {
      g = fmaf(g, y, sp[p][tid] * inv_int(p + 1));
      e = fmaf(e, y, sp[p][tid]);
    }
    for (int r = 0; r < s; ++r) {
      gm[tid] = g;
      em[tid] = e;
      __syncthreads();
      float ge = 0.0f, ee = 0.0f;
#pragma unroll
      for (int c = 0; c < 16; ++c) {
        ge = fmaf(gm[i * 16 + c], em[c * 16 + j], ge);
        ee = fmaf(em[i * 16 + c], em[c * 16 + j], ee);
      }
      __syncthreads();
      g = 0.5f * (ge + g);
      e = ee;
    }
    gm[tid] = g;
    __syncthreads();
    if (tid < 16) {
      float acc = 0.0f;
#pragma unroll
      for (int c = 0; c < 16; ++c) acc = fmaf(gm[tid * 16 + c], vv[c], acc);
      a.loc[((size_t)b * a.n_int + t) * a.LW + tid] = tid < a.d ? acc : 0.0f;
    }
    __syncthreads();
  }
}

// Adjoint of s1 = phi(X) v, X = -h A, for the level-1 cotangent g of every interval (read from loc, then zeroed
// there, so that the series leaf's adjoint that follows sees level 2 only):
//   dv = phi(X)^T g,  dX = Gam = int_0^1 int_0^s e^{(s-r) X^T} g v^T e^{r X^T} dr ds,  dA += -h Gam,
//   dh = -<A, Gam>.
// Gam is the upper block of phi(Z) for the block-triangular Z = [[X^T, g v^T], [0, X^T]] (the Frechet derivative
// of phi; its diagonal blocks are phi(X^T)), evaluated on Z / 2^s (the same s as the forward) by Horner over the
// blocks, G_p = I / (p+1)! + Z G_{p+1} (P G_d = g (G_d^T v)^T stays a rank-one update), E = I + Z G, then s
// doublings on the blocks: G <- G (E + I) / 2, E <- E E. Per-interval dv and dh go to dv1 / dh1 (added after the
// series adjoint), -h Gam summed per workgroup into part (a fixed-order sum in k_bs_dA).
__global__ __launch_bounds__(256) void k_bs_level1_bwd(Args a, float* __restrict__ dv1, float* __restrict__ dh1,
                                                       float* __restrict__ part) {
  __shared__ float at[256];  // A^T (padded)
  __shared__ float yt[256], gd[256], gu[256], ed[256], eu[256];
  __shared__ float gv[16], vv[16], w[16];
  __shared__ float red[256];
  const int tid = threadIdx.x, i = tid >> 4, j = tid & 15;
  at[tid] = a.apow[256 + j * 16 + i];  // P_1 = A
  const float norm1 = a.apow[a.npow * 256];
  float dA = 0.0f;
  __syncthreads();
  const long total = (long)a.B * a.n_int;
  for (long it = blockIdx.x; it < total; it += gridDim.x) {
    const int b = (int)(it / a.n_int), t = (int)(it - (long)b * a.n_int);
    const float* th = a.clock + (size_t)b * a.L;
    const float h = th[t + 1] - th[t];
    float* row = a.loc + ((size_t)b * a.n_int + t) * a.LW;
    if (tid < 16) {
      const float* x = a.path + ((size_t)b * a.L + t) * a.d;
      vv[tid] = tid < a.d ? x[a.d + tid] - x[tid] : 0.0f;
      gv[tid] = tid < a.d ? row[tid] : 0.0f;
    }
    int s = 0;
    float xn = fabsf(h) * norm1;
    while (xn > 1.0f && s < SQMAX) {
      xn *= 0.5f;
      ++s;
    }
    const float scl = ldexpf(1.0f, -s), y = -h * scl;
    yt[tid] = y * at[tid];
    if (tid < 16) row[tid] = 0.0f;  // the series adjoint sees no level-1 cotangent (gv holds it)
    // Horner start: G_PM = I / (PM + 1)!
    float cfac = 1.0f;
    for (int p = 2; p <= PM + 1; ++p) cfac *= inv_int(p);
    gd[tid] = i == j ? cfac : 0.0f;
    gu[tid] = 0.0f;
    __syncthreads();
    for (int p = PM - 1; p >= -1; --p) {  // p = -1: E = I + Z G
      if (tid < 16) {
        float acc = 0.0f;
#pragma unroll
        for (int k = 0; k < 16; ++k) acc = fmaf(vv[k], gd[k * 16 + tid], acc);
        w[tid] = acc;
      }
      __syncthreads();
      float nd = 0.0f, nu = 0.0f;
#pragma unroll
      for (int c = 0; c < 16; ++c) {
        nd = fmaf(yt[i * 16 + c], gd[c * 16 + j], nd);
        nu = fmaf(yt[i * 16 + c], gu[c * 16 + j], nu);
      }
      nu = fmaf(scl * gv[i], w[j], nu);
      if (p >= 0) {
        float c = 1.0f;  // 1 / (p + 1)!
        for (int m = 2; m <= p + 1; ++m) c *= inv_int(m);
        nd += i == j ? c : 0.0f;
        __syncthreads();
        gd[tid] = nd;
        gu[tid] = nu;
      } else {
        nd += i == j ? 1.0f : 0.0f;
        __syncthreads();
        ed[tid] = nd;
        eu[tid] = nu;
      }
      __syncthreads();
    }
    for (int r = 0; r < s; ++r) {
      float g_e = 0.0f, g_eu = 0.0f, u_e = 0.0f, e_e = 0.0f, e_eu = 0.0f, eu_e = 0.0f;
#pragma unroll
      for (int c = 0; c < 16; ++c) {
        const float gdic = gd[i * 16 + c], guic = gu[i * 16 + c], edic = ed[i * 16 + c], euic = eu[i * 16 + c];
        const float edcj = ed[c * 16 + j], eucj = eu[c * 16 + j];
        g_e = fmaf(gdic, edcj, g_e);
        g_eu = fmaf(gdic, eucj, g_eu);
        u_e = fmaf(guic, edcj, u_e);
        e_e = fmaf(edic, edcj, e_e);
        e_eu = fmaf(edic, eucj, e_eu);
        eu_e = fmaf(euic, edcj, eu_e);
      }
      const float ngd = 0.5f * (g_e + gd[tid]), ngu = 0.5f * (g_eu + u_e + gu[tid]);
      __syncthreads();
      gd[tid] = ngd;
      gu[tid] = ngu;
      ed[tid] = e_e;
      eu[tid] = e_eu + eu_e;
      __syncthreads();
    }
    // gd = phi(X^T), gu = Gam
    const float gam = gu[tid];
    dA = fmaf(-h, gam, dA);
    red[tid] = at[j * 16 + i] * gam;  // A[i][j] Gam[i][j]
    __syncthreads();
    for (int o = 128; o >= 1; o >>= 1) {
      if (tid < o) red[tid] += red[tid + o];
      __syncthreads();
    }
    if (tid < 16) {
      float acc = 0.0f;
#pragma unroll
      for (int k = 0; k < 16; ++k) acc = fmaf(gd[tid * 16 + k], gv[k], acc);
      dv1[it * 16 + tid] = acc;
    }
    if (tid == 0) dh1[it] = -red[0];
    __syncthreads();
  }
  part[(size_t)blockIdx.x * 256 + tid] = dA;
}

// the level-1 shares of dv and dh added to the series adjoint's (which wrote o.dv / o.dh)
__global__ void k_bs_add(Args a, LeafBwd o, const float* __restrict__ dv1, const float* __restrict__ dh1) {
  const long total = (long)a.B * a.n_int;
  for (long e = (long)blockIdx.x * blockDim.x + threadIdx.x; e < total * 17; e += (long)gridDim.x * blockDim.x) {
    if (e < total * 16) o.dv[e] += dv1[e];
    else o.dh[e - total * 16] += dh1[e - total * 16];
  }
}

// grad_A += the workgroups' -h Gam sums, in a fixed order (float64)
__global__ __launch_bounds__(256) void k_bs_dA(Args a, const float* __restrict__ part, int nparts, float* grad_A) {
  const int tid = threadIdx.x, i = tid >> 4, j = tid & 15;
  double acc = 0.0;
  for (int w = 0; w < nparts; ++w) acc += (double)part[(size_t)w * 256 + tid];
  if (i < a.d && j < a.d) grad_A[i * a.d + j] += (float)acc;
}

// knot cotangents: dpath[k] = dv_{k-1} - dv_k, dclock[k] = dh_{k-1} - dh_k, plus the shared steps of the cached modes
// (the flow step th[1] - th[0], or th[2] - th[1] for the basepoint mode; the Van Loan step likewise)
__global__ void k_knots(Args a, LeafBwd o, float* grad_path, float* grad_clock) {
  const int b = blockIdx.y;
  const int k = blockIdx.x * blockDim.x + threadIdx.x;
  if (k >= a.L) return;
  const size_t base = (size_t)b * a.n_int;
  for (int r = 0; r < a.d; ++r) {
    const float lo = k > 0 ? o.dv[(base + k - 1) * 16 + r] : 0.0f;
    const float hi = k < a.n_int ? o.dv[(base + k) * 16 + r] : 0.0f;
    grad_path[((size_t)b * a.L + k) * a.d + r] = lo - hi;
  }
  if (grad_clock) {
    float v = (k > 0 ? o.dh[base + k - 1] : 0.0f) - (k < a.n_int ? o.dh[base + k] : 0.0f);
    const float sf = o.dsh[2 * b], sv = o.dsh[2 * b + 1];
    if (a.flow_mode == EWS_FLOW_CACHED) v += (k == 1 ? sf : 0.0f) - (k == 0 ? sf : 0.0f);
    if (a.flow_mode == EWS_FLOW_CACHED_BASEPOINT) v += (k == 2 ? sf : 0.0f) - (k == 1 ? sf : 0.0f);
    if (a.leaf == EWS_LEAF_VAN_LOAN && a.vl_mode == EWS_FLOW_CACHED) v += (k == 1 ? sv : 0.0f) - (k == 0 ? sv : 0.0f);
    if (a.leaf == EWS_LEAF_VAN_LOAN && a.vl_mode == EWS_FLOW_CACHED_BASEPOINT)
      v += (k == 2 ? sv : 0.0f) - (k == 1 ? sv : 0.0f);
    grad_clock[(size_t)b * a.L + k] = v;
  }
}

// ------------------------------------------------------------------------------------------------ readouts
// zero state rows (carries row 0)
__global__ void k_zero_rows(float* base, long stride, int n_rows, int width) {
  const int r = blockIdx.y;
  if (r >= n_rows) return;
  for (int e = blockIdx.x * blockDim.x + threadIdx.x; e < width; e += gridDim.x * blockDim.x)
    base[(long)r * stride + e] = 0.0f;
}
// terminal row: the carry after the last chunk, unpadded, with the level-0 column
__global__ void k_terminal(Args a) {
  const int b = blockIdx.y;
  const float* src = a.car + ((size_t)b * (a.C + 1) + a.C) * a.LW;
  float* o = a.out + (size_t)b * a.W;
  if (a.lvl0 && blockIdx.x == 0 && threadIdx.x == 0) o[0] = 1.0f;
  for (int e = blockIdx.x * blockDim.x + threadIdx.x; e < a.LW; e += gridDim.x * blockDim.x) {
    const long oi = out_index(a.N, a.d, e);
    if (oi >= 0) o[a.lvl0 + oi] = src[e];
  }
}
// mean / max over the prefix rows (ews/layer.py:261-264), per output column
__global__ void k_reduce(Args a) {
  const int b = blockIdx.y;
  const int col = blockIdx.x * blockDim.x + threadIdx.x;
  if (col >= a.W) return;
  const float* p = a.pre + (size_t)b * a.n_int * a.W + col;
  float acc = a.readout == EWS_READOUT_MAX ? p[0] : 0.0f;
  for (int t = 0; t < a.n_int; ++t) {
    const float v = p[(size_t)t * a.W];
    acc = a.readout == EWS_READOUT_MAX ? fmaxf(acc, v) : acc + v;
  }
  a.out[(size_t)b * a.W + col] = a.readout == EWS_READOUT_MAX ? acc : acc / (float)a.n_int;
}
// given levels (B, n, D) packed and flows (B, n, d, d) -> padded loc / fl (the combine-only entry point)
__global__ void k_pad_inputs(Args a, const float* levels, const float* flows) {
  const long it = blockIdx.x;
  const int b = (int)(it / a.n_int), t = (int)(it - (long)b * a.n_int);
  const int D = a.W - a.lvl0;
  const float* lv = levels + ((size_t)b * a.n_int + t) * D;
  float* lo = a.loc + ((size_t)b * a.n_int + t) * a.LW;
  for (int e = threadIdx.x; e < a.LW; e += blockDim.x) {
    const long oi = out_index(a.N, a.d, e);
    lo[e] = oi >= 0 ? lv[oi] : 0.0f;
  }
  const float* fi = flows + ((size_t)b * a.n_int + t) * a.d * a.d;
  float* fo = a.fl + ((size_t)b * a.n_int + t) * 256;
  for (int e = threadIdx.x; e < 256; e += blockDim.x) {
    const int i = e >> 4, j = e & 15;
    fo[e] = (i < a.d && j < a.d) ? fi[i * a.d + j] : (i == j ? 1.0f : 0.0f);
  }
}
// padded loc / fl -> packed levels (B, n, D) and flows (B, n, d, d) (the leaf-only entry point)
__global__ void k_unpad_outputs(Args a, float* levels, float* flows) {
  const long it = blockIdx.x;
  const int b = (int)(it / a.n_int), t = (int)(it - (long)b * a.n_int);
  const int D = a.W - a.lvl0;
  const float* lo = a.loc + ((size_t)b * a.n_int + t) * a.LW;
  float* lv = levels + ((size_t)b * a.n_int + t) * D;
  for (int e = threadIdx.x; e < a.LW; e += blockDim.x) {
    const long oi = out_index(a.N, a.d, e);
    if (oi >= 0) lv[oi] = lo[e];
  }
  const float* fo = a.fl + ((size_t)b * a.n_int + t) * 256;
  float* fi = flows + ((size_t)b * a.n_int + t) * a.d * a.d;
  for (int e = threadIdx.x; e < 256; e += blockDim.x) {
    const int i = e >> 4, j = e & 15;
    if (i < a.d && j < a.d) fi[i * a.d + j] = fo[e];
  }
}

// Token cache (ews/core/token_scan.py:91-118): step (b, t) reads the cache row of its token, the packed levels
// P_cache[g] (ews/core/chen_scan.py:33-46) and the flow D_cache[g]; a padded step is the unit signature (zero levels)
// with the identity flow. Token ids are clamped to [0, V) (the clamping of an out-of-range JAX gather).
// One wavefront per step, four steps per workgroup (a workgroup per step left the chip scheduling tiny workgroups).
__global__ __launch_bounds__(256) void k_pad_tokens(Args a, const int* tok, const uint8_t* mask, const float* pc,
                                                    const float* dc, int V, int D) {
  const long it = (long)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (it >= (long)a.B * a.n_int) return;
  const bool on = mask == nullptr || mask[it] != 0;
  const int g = min(max(tok[it], 0), V - 1);
  const float* lv = pc + (size_t)g * D;
  float* lo = a.loc + it * a.LW;
  for (int e = lane; e < a.LW; e += 64) {
    const long oi = out_index(a.N, a.d, e);
    lo[e] = (on && oi >= 0) ? lv[oi] : 0.0f;
  }
  const float* fi = dc + (size_t)g * a.d * a.d;
  float* fo = a.fl + it * 256;
  for (int e = lane; e < 256; e += 64) {
    const int i = e >> 4, j = e & 15;
    fo[e] = (on && i < a.d && j < a.d) ? fi[i * a.d + j] : (i == j ? 1.0f : 0.0f);
  }
}

// Cache gradients: the per-step cotangents (ds_t in loc, dM_t in fl, padded) summed by token. Stage 1: a
// workgroup per (256 columns, chunk of kTokChunk steps, group of 16 tokens), each thread owning one column of the
// 16 accumulators and reading 8 steps ahead; stage 2: per (token, column) the chunks summed by 4 wavefronts and
// combined in a fixed order, then unpadded. Deterministic.
constexpr int kTokChunk = 512;
__global__ __launch_bounds__(256) void k_token_grads1(Args a, const int* tok, const uint8_t* mask, int V,
                                                      float* part) {
  __shared__ float acc[16][256];
  const int E = a.LW + 256;
  const int col = blockIdx.x * 256 + threadIdx.x;
  const int ch = blockIdx.y, g0 = blockIdx.z * 16;
  const long P = (long)a.B * a.n_int;
  const long p0 = (long)ch * kTokChunk, p1 = min(P, p0 + kTokChunk);
  for (int k = 0; k < 16; ++k) acc[k][threadIdx.x] = 0.0f;
  if (col >= E) return;  // no barrier below: each thread owns its column
  const bool isloc = col < a.LW;
  const float* src = isloc ? a.loc + col : a.fl + (col - a.LW);
  const long stride = isloc ? a.LW : 256;
  long pos = p0;
  for (; pos + 8 <= p1; pos += 8) {
    float v[8];
    int g[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const long pp = pos + k;
      const bool on = mask == nullptr || mask[pp] != 0;
      g[k] = on ? min(max(tok[pp], 0), V - 1) - g0 : -1;
      v[k] = src[pp * stride];
    }
#pragma unroll
    for (int k = 0; k < 8; ++k)
      if (g[k] >= 0 && g[k] < 16) acc[g[k]][threadIdx.x] += v[k];
  }
  for (; pos < p1; ++pos) {
    if (mask != nullptr && mask[pos] == 0) continue;
    const int g = min(max(tok[pos], 0), V - 1) - g0;
    if (g >= 0 && g < 16) acc[g][threadIdx.x] += src[pos * stride];
  }
  for (int k = 0; k < 16 && g0 + k < V; ++k) part[((size_t)ch * V + g0 + k) * E + col] = acc[k][threadIdx.x];
}

__global__ __launch_bounds__(256) void k_token_grads2(Args a, const float* part, int nch, int V, int D, float* gP,
                                                      float* gD) {
  __shared__ double red[4][64];
  const int E = a.LW + 256;
  const int l = threadIdx.x & 63, w = threadIdx.x >> 6;
  const long idx = (long)blockIdx.x * 64 + l;
  const bool ok = idx < (long)V * E;
  double s0 = 0.0, s1 = 0.0;
  if (ok) {
    int c = w;
    for (; c + 4 < nch; c += 8) {
      s0 += part[(size_t)c * V * E + idx];
      s1 += part[(size_t)(c + 4) * V * E + idx];
    }
    if (c < nch) s0 += part[(size_t)c * V * E + idx];
  }
  red[w][l] = s0 + s1;
  __syncthreads();
  if (w != 0 || !ok) return;
  const double s = (red[0][l] + red[1][l]) + (red[2][l] + red[3][l]);
  const int g = (int)(idx / E), e = (int)(idx - (long)g * E);
  if (e < a.LW) {
    const long oi = out_index(a.N, a.d, e);
    if (oi >= 0) gP[(size_t)g * D + oi] = (float)s;
  } else {
    const int f = e - a.LW, i = f >> 4, j = f & 15;
    if (i < a.d && j < a.d) gD[((size_t)g * a.d + i) * a.d + j] = (float)s;
  }
}

// first row index of the column maximum over the prefix rows (B, n, Wr) (the max readout's cotangent goes there)
__global__ void k_argmax(const float* rows, int n, int Wr, int* amax) {
  const int b = blockIdx.y;
  const int col = blockIdx.x * blockDim.x + threadIdx.x;
  if (col >= Wr) return;
  const float* p = rows + (size_t)b * n * Wr + col;
  float best = p[0];
  int arg = 0;
  for (int t = 1; t < n; ++t) {
    const float v = p[(size_t)t * Wr];
    if (v > best) {
      best = v;
      arg = t;
    }
  }
  amax[(size_t)b * Wr + col] = arg;
}
// row C of the adjoint carries: the terminal readout's cotangent (padded, without the level-0 column), or zero
__global__ void k_lam_end(Args a, const float* gterm, int glvl0) {
  const int b = blockIdx.y;
  float* o = a.lam + ((size_t)b * (a.C + 1) + a.C) * a.LW;
  for (int e = blockIdx.x * blockDim.x + threadIdx.x; e < a.LW; e += gridDim.x * blockDim.x) {
    const long oi = out_index(a.N, a.d, e);
    o[e] = (gterm && oi >= 0) ? gterm[(size_t)b * a.W + glvl0 + oi] : 0.0f;
  }
}

}  // namespace dense
}  // namespace ews

// ================================================================================================= C ABI
namespace {

using namespace ews::dense;

size_t al256(size_t x) { return (x + 255) & ~(size_t)255; }

// The forward's carry scan over the chunk summaries runs in blocks of kCarryBlock chunks when there are at least
// two blocks (NBc of them): block summaries, a scan over the blocks, then each block from its carry.
constexpr int kCarryBlock = 8;
struct DPlan {
  int B, L, n_int, d, N, q, QB, T, C, LW, D, W, npow;
  int leaf, vm, vl_expm, vl_mode, chen_expm;
  int NBc;  // carry-scan blocks per sample (0: one pass over the chunk summaries)
};

int dense_plan(const ews_dense_desc* s, DPlan& p) {
  if (!s) return EWS_ERR_NULL;
  if (s->depth < 1 || s->depth > 3) return EWS_ERR_DEPTH;
  if (s->flow_mode < 0 || s->flow_mode > 2) return EWS_ERR_OPTION;
  if (s->readout < 0 || s->readout > 3) return EWS_ERR_OPTION;
  if (s->batch < 1 || s->length < 2 || s->dim < 1 || s->dim > 16) return EWS_ERR_SHAPE;
  if (s->leaf != EWS_LEAF_SERIES && s->leaf != EWS_LEAF_VAN_LOAN && s->leaf != EWS_LEAF_BLOCK_SERIES)
    return EWS_ERR_OPTION;
  if (s->leaf == EWS_LEAF_BLOCK_SERIES && s->depth > 2) return EWS_ERR_DEPTH;
  const bool vl = s->leaf == EWS_LEAF_VAN_LOAN;
  if (!vl && (s->series_q < 0 || s->series_q > QMAX)) return EWS_ERR_OPTION;
  if (vl && (s->vl_steps < 1 || s->vl_steps > 64)) return EWS_ERR_OPTION;
  if (vl && (s->vl_expm < 0 || s->vl_expm > 3 || s->vl_mode < 0 || s->vl_mode > 2)) return EWS_ERR_OPTION;
  if (s->chen_expm < 0 || s->chen_expm > 3) return EWS_ERR_OPTION;
  if (s->flow_mode == EWS_FLOW_CACHED_BASEPOINT && s->length < 3) return EWS_ERR_SHAPE;
  if (vl && s->vl_mode == EWS_FLOW_CACHED_BASEPOINT && s->length < 3) return EWS_ERR_SHAPE;
  if (s->chunk < 0) return EWS_ERR_SHAPE;
  p.leaf = s->leaf;
  p.vm = vl ? s->vl_steps : 0;
  p.vl_expm = vl ? s->vl_expm : 0;
  p.vl_mode = vl ? s->vl_mode : 0;
  p.chen_expm = s->chen_expm;
  p.B = s->batch;
  p.L = s->length;
  p.n_int = p.L - 1;
  p.d = s->dim;
  p.N = s->depth;
  p.q = vl ? 0 : s->series_q;
  p.QB = p.q <= 4 ? 4 : p.q <= 8 ? 8 : p.q <= 12 ? 12 : p.q <= 16 ? 16 : p.q <= 20 ? 20 : p.q <= 24 ? 24
       : p.q <= 32 ? 32 : 40;
  p.T = s->chunk ? s->chunk : 64;
  p.C = (p.n_int + p.T - 1) / p.T;
  p.NBc = p.C >= 2 * kCarryBlock ? (p.C + kCarryBlock - 1) / kCarryBlock : 0;
  p.LW = lw_of(p.N);
  p.D = 0;
  for (int k = 1, m = 1; k <= p.N; ++k) {
    m *= p.d;
    p.D += m;
  }
  p.W = p.D + (s->level0 ? 1 : 0);
  p.npow = (p.q > PM ? p.q : PM) + 1;
  return EWS_OK;
}

constexpr int kLeafBwdBlocks = 1024;  // workgroups of the leaf adjoint (one partial dA set each)

struct DWs {
  size_t apow, loc, fl, summ, sfl, car, pre, mats, bsumm, bsfl, bcar, lloc, lam, bagg, bl, amax, dv, dh, dsh, dshi,
      part, hsum, vlsave;
  size_t bsdv, bsdh, bspart, total;  // block-series level 1: per-interval dv / dh and the workgroups' dA sums
};
// bwd: the backward's layout, the forward's buffers (prefix rows always) followed by the adjoint scan's
DWs dense_ws(const DPlan& p, int readout, bool bwd = false) {
  DWs w{};
  size_t off = 0;
  const size_t BC = (size_t)p.B * p.C, BN = (size_t)p.B * p.n_int;
  w.apow = off; off += al256(((size_t)p.npow * 256 + 1) * 4);
  w.loc = off; off += al256(BN * p.LW * 4);
  w.fl = off; off += al256(BN * 256 * 4);
  w.summ = off; off += al256(BC * p.LW * 4);
  w.sfl = off; off += al256(BC * 256 * 4);
  w.car = off; off += al256((size_t)p.B * (p.C + 1) * p.LW * 4);
  w.pre = off;
  off += bwd ? al256(BN * p.LW * 4)
             : (readout == EWS_READOUT_MEAN || readout == EWS_READOUT_MAX) ? al256(BN * p.W * 4) : 0;
  w.mats = off; off += al256((size_t)p.B * 768 * 4);
  w.bsumm = off; off += al256((size_t)p.B * p.NBc * p.LW * 4);
  w.bsfl = off; off += al256((size_t)p.B * p.NBc * 256 * 4);
  w.bcar = off; off += p.NBc ? al256((size_t)p.B * (p.NBc + 1) * p.LW * 4) : 0;
  if (bwd) {
    w.lloc = off; off += al256(BC * p.LW * 4);
    w.lam = off; off += al256((size_t)p.B * (p.C + 1) * p.LW * 4);
    w.bagg = off; off += al256((size_t)p.B * p.NBc * p.LW * 4);
    w.bl = off; off += p.NBc ? al256((size_t)p.B * (p.NBc + 1) * p.LW * 4) : 0;
    w.amax = off; off += al256((size_t)p.B * p.LW * 4);
    w.dv = off; off += al256(BN * 16 * 4);
    w.dh = off; off += al256(BN * 4);
    w.dsh = off; off += al256((size_t)p.B * 2 * 4);
    w.dshi = off; off += al256(BN * 2 * 4);
    w.part = off; off += al256((size_t)kLeafBwdBlocks * (HP + 1) * 256 * 4);
    w.hsum = off; off += al256((size_t)PRS * (HP + 1) * 256 * 8);
    w.vlsave = off; off += p.leaf == EWS_LEAF_VAN_LOAN ? al256(BN * (512 + 16 * (size_t)p.vm) * 4) : 0;
    const bool bs = p.leaf == EWS_LEAF_BLOCK_SERIES;
    w.bsdv = off; off += bs ? al256(BN * 16 * 4) : 0;
    w.bsdh = off; off += bs ? al256(BN * 4) : 0;
    w.bspart = off; off += bs ? al256((size_t)kLeafBwdBlocks * 256 * 4) : 0;
  }
  w.total = off;
  return w;
}

Args dense_args(const ews_dense_desc* s, const DPlan& p, const float* path, const float* clock, const float* A,
                float* out, void* workspace, bool bwd = false) {
  Args a{};
  a.B = p.B; a.L = p.L; a.n_int = p.n_int; a.d = p.d; a.N = p.N; a.q = p.q;
  a.flow_mode = s->flow_mode; a.readout = s->readout; a.lvl0 = s->level0 ? 1 : 0; a.W = p.W; a.LW = p.LW;
  a.T = p.T; a.C = p.C; a.npow = p.npow;
  a.leaf = p.leaf; a.vm = p.vm; a.vl_expm = p.vl_expm; a.vl_mode = p.vl_mode; a.chen_expm = p.chen_expm;
  a.path = path; a.clock = clock; a.A = A; a.out = out;
  const DWs w = dense_ws(p, s->readout, bwd);
  char* ws = (char*)workspace;
  a.apow = (float*)(ws + w.apow); a.loc = (float*)(ws + w.loc); a.fl = (float*)(ws + w.fl);
  a.summ = (float*)(ws + w.summ); a.sfl = (float*)(ws + w.sfl); a.car = (float*)(ws + w.car);
  a.pre = (float*)(ws + w.pre); a.mats = (float*)(ws + w.mats);
  a.bsumm = (float*)(ws + w.bsumm); a.bsfl = (float*)(ws + w.bsfl); a.bcar = (float*)(ws + w.bcar);
  if (bwd) {
    a.lloc = (float*)(ws + w.lloc); a.lam = (float*)(ws + w.lam); a.amax = (int*)(ws + w.amax);
    a.bagg = (float*)(ws + w.bagg); a.bl = (float*)(ws + w.bl);
    a.vlsave = p.leaf == EWS_LEAF_VAN_LOAN ? (float*)(ws + w.vlsave) : nullptr;
  }
  return a;
}

#define DENSE_CHECK()                                          \
  do {                                                         \
    if (hipGetLastError() != hipSuccess) return EWS_ERR_LAUNCH; \
  } while (0)

int launch_local(const DPlan& p, const Args& a, hipStream_t st) {
  const long total = (long)p.B * p.n_int;
  const int grid = (int)(total < 4096 ? total : 4096);
#define EWS_LOCAL(NN, QQ) hipLaunchKernelGGL((k_local<NN, QQ>), dim3(grid), dim3(256), 0, st, a)
#define EWS_LOCAL_Q(NN)                          \
  switch (p.QB) {                                \
    case 4: EWS_LOCAL(NN, 4); break;             \
    case 8: EWS_LOCAL(NN, 8); break;             \
    case 12: EWS_LOCAL(NN, 12); break;           \
    case 16: EWS_LOCAL(NN, 16); break;           \
    case 20: EWS_LOCAL(NN, 20); break;           \
    case 24: EWS_LOCAL(NN, 24); break;           \
    case 32: EWS_LOCAL(NN, 32); break;           \
    default: EWS_LOCAL(NN, 40); break;           \
  }
  if (p.N == 1) { EWS_LOCAL_Q(1) }
  else if (p.N == 2) { EWS_LOCAL_Q(2) }
  else {
    const int grid3 = (int)((total + 3) / 4 < 2048 ? (total + 3) / 4 : 2048);
#define EWS_LOCAL3(QQ) hipLaunchKernelGGL((k_local3<QQ>), dim3(grid3), dim3(256), 0, st, a)
    switch (p.QB) {
      case 4: EWS_LOCAL3(4); break;
      case 8: EWS_LOCAL3(8); break;
      case 12: EWS_LOCAL3(12); break;
      case 16: EWS_LOCAL3(16); break;
      case 20: EWS_LOCAL3(20); break;
      case 24: EWS_LOCAL3(24); break;
      case 32: EWS_LOCAL3(32); break;
      default: EWS_LOCAL3(40); break;
    }
#undef EWS_LOCAL3
  }
#undef EWS_LOCAL_Q
#undef EWS_LOCAL
  DENSE_CHECK();
  return EWS_OK;
}

template <bool SUMMARY>
int launch_scan(int N, const Seq& s, dim3 grid, hipStream_t st) {
  if (N == 3) hipLaunchKernelGGL((k_scan<3, SUMMARY>), grid, dim3(256), 0, st, s);
  else if (N == 2) hipLaunchKernelGGL((k_scan<2, SUMMARY>), grid, dim3(64), 0, st, s);
  else hipLaunchKernelGGL((k_scan<1, SUMMARY>), grid, dim3(64), 0, st, s);
  DENSE_CHECK();
  return EWS_OK;
}

// passes 1..3 (combine): summaries, carries, outputs
int dense_combine_pass(const ews_dense_desc* s, const DPlan& p, const Args& a, hipStream_t st, int pass) {
  switch (pass) {
    case 1: {
      Seq q{};
      q.lv = a.loc; q.lv_bs = (long)p.n_int * p.LW; q.fl = a.fl; q.fl_bs = (long)p.n_int * 256;
      q.n = p.n_int; q.T = p.T; q.summ = a.summ; q.sfl = a.sfl; q.C = p.C; q.d = p.d;
      return launch_scan<true>(p.N, q, dim3(p.C, p.B), st);
    }
    case 2: {
      hipLaunchKernelGGL(k_zero_rows, dim3(1, p.B), dim3(256), 0, st, a.car, (long)(p.C + 1) * p.LW, p.B, p.LW);
      DENSE_CHECK();
      if (p.NBc) {  // blocks of kCarryBlock chunks: a chain of 3 kCarryBlock-ish steps instead of C
        const int G = kCarryBlock, NB = p.NBc;
        Seq q1{};  // block summaries: the SUMMARY scan over the chunk summaries
        q1.lv = a.summ; q1.lv_bs = (long)p.C * p.LW; q1.fl = a.sfl; q1.fl_bs = (long)p.C * 256;
        q1.n = p.C; q1.T = G; q1.summ = a.bsumm; q1.sfl = a.bsfl; q1.C = NB; q1.d = p.d;
        int rc = launch_scan<true>(p.N, q1, dim3(NB, p.B), st);
        if (rc != EWS_OK) return rc;
        hipLaunchKernelGGL(k_zero_rows, dim3(1, p.B), dim3(256), 0, st, a.bcar, (long)(NB + 1) * p.LW, p.B, p.LW);
        DENSE_CHECK();
        Seq q2{};  // block carries: one pass over the block summaries of each sample
        q2.lv = a.bsumm; q2.lv_bs = (long)NB * p.LW; q2.fl = a.bsfl; q2.fl_bs = (long)NB * 256;
        q2.n = NB; q2.T = NB; q2.rows = a.bcar + p.LW; q2.rows_bs = (long)(NB + 1) * p.LW; q2.rows_ld = p.LW;
        q2.padded = 1; q2.lvl0 = 0; q2.d = p.d; q2.C = 1;
        rc = launch_scan<false>(p.N, q2, dim3(1, p.B), st);
        if (rc != EWS_OK) return rc;
        Seq q3{};  // chunk carries: each block from its carry
        q3.lv = a.summ; q3.lv_bs = (long)p.C * p.LW; q3.fl = a.sfl; q3.fl_bs = (long)p.C * 256;
        q3.n = p.C; q3.T = G; q3.init = a.bcar; q3.init_bs = (long)(NB + 1) * p.LW;
        q3.rows = a.car + p.LW; q3.rows_bs = (long)(p.C + 1) * p.LW; q3.rows_ld = p.LW;
        q3.padded = 1; q3.lvl0 = 0; q3.d = p.d; q3.C = NB;
        return launch_scan<false>(p.N, q3, dim3(NB, p.B), st);
      }
      Seq q{};
      q.lv = a.summ; q.lv_bs = (long)p.C * p.LW; q.fl = a.sfl; q.fl_bs = (long)p.C * 256;
      q.n = p.C; q.T = p.C; q.rows = a.car + p.LW; q.rows_bs = (long)(p.C + 1) * p.LW; q.rows_ld = p.LW;
      q.padded = 1; q.lvl0 = 0; q.d = p.d; q.C = 1;
      return launch_scan<false>(p.N, q, dim3(1, p.B), st);
    }
    case 3: {
      if (s->readout == EWS_READOUT_TERMINAL) {
        hipLaunchKernelGGL(k_terminal, dim3((p.LW + 255) / 256, p.B), dim3(256), 0, st, a);
        DENSE_CHECK();
        return EWS_OK;
      }
      const bool red = s->readout != EWS_READOUT_PREFIX;
      Seq q{};
      q.lv = a.loc; q.lv_bs = (long)p.n_int * p.LW; q.fl = a.fl; q.fl_bs = (long)p.n_int * 256;
      q.n = p.n_int; q.T = p.T; q.init = a.car; q.init_bs = (long)(p.C + 1) * p.LW;
      q.rows = red ? a.pre : a.out; q.rows_bs = (long)p.n_int * p.W; q.rows_ld = p.W; q.padded = 0;
      q.lvl0 = red ? 1 : (s->level0 ? 1 : 0); q.d = p.d; q.C = p.C;
      if (red && !s->level0) return EWS_ERR_OPTION;  // mean / max rows carry the level-0 column
      const int rc = launch_scan<false>(p.N, q, dim3(p.C, p.B), st);
      if (rc != EWS_OK || !red) return rc;
      hipLaunchKernelGGL(k_reduce, dim3((p.W + 255) / 256, p.B), dim3(256), 0, st, a);
      DENSE_CHECK();
      return EWS_OK;
    }
    default:
      return EWS_ERR_OPTION;
  }
}

// the Van Loan leaf (levels and flows), or the flows of a scheme other than the series kernels' fused exact ones
int launch_vl_and_flows(const DPlan& p, const Args& a, hipStream_t st) {
  const bool vl = p.leaf == EWS_LEAF_VAN_LOAN;
  const long total = (long)p.B * p.n_int;
  const bool prep = (vl && p.vl_mode != EWS_FLOW_PER_INTERVAL) ||
                    (a.flow_mode != EWS_FLOW_PER_INTERVAL && (vl || p.chen_expm != EWS_EXPM_EXACT));
  if (prep) {
    hipLaunchKernelGGL(k_prep, dim3(p.B), dim3(64), 0, st, a);
    DENSE_CHECK();
  }
  if (vl) {
    const size_t table = (size_t)(PM + 1) * 256 * 4, region = (size_t)vl_region(p.vm) * 4;
    const int nw = table + 4 * region <= 65536 ? 4 : 2;
    const long blocks = (total + nw - 1) / nw;
    const int grid = (int)(blocks < 8192 ? blocks : 8192);
    const size_t shm = table + nw * region;
    const bool ex = p.chen_expm == EWS_EXPM_EXACT;
#define EWS_VL(NN)                                                                                   \
  do {                                                                                               \
    if (ex) hipLaunchKernelGGL((k_vl<NN, true>), dim3(grid), dim3(64 * nw), shm, st, a);            \
    else hipLaunchKernelGGL((k_vl<NN, false>), dim3(grid), dim3(64 * nw), shm, st, a);              \
  } while (0)
    if (p.N == 1) EWS_VL(1);
    else if (p.N == 2) EWS_VL(2);
    else EWS_VL(3);
#undef EWS_VL
    DENSE_CHECK();
  }
  if (!vl && p.chen_expm != EWS_EXPM_EXACT) {  // the Van Loan kernel writes its flows itself
    const long blocks = (total + 3) / 4;
    const int grid = (int)(blocks < 8192 ? blocks : 8192);
    hipLaunchKernelGGL(k_flows, dim3(grid), dim3(256), 0, st, a);
    DENSE_CHECK();
  }
  return EWS_OK;
}

int dense_forward_pass(const ews_dense_desc* s, const DPlan& p, const Args& a, hipStream_t st, int pass) {
  if (pass == 0) {
    hipLaunchKernelGGL(k_powers, dim3(1), dim3(256), 0, st, a);
    DENSE_CHECK();
    if (p.leaf != EWS_LEAF_VAN_LOAN) {  // the series letters (block series: level 2; level 1 overwritten next)
      const int rc = launch_local(p, a, st);
      if (rc != EWS_OK) return rc;
    }
    if (p.leaf == EWS_LEAF_BLOCK_SERIES) {
      const long total = (long)p.B * p.n_int;
      hipLaunchKernelGGL(k_bs_level1, dim3((unsigned)(total < 8192 ? total : 8192)), dim3(256), 0, st, a);
      DENSE_CHECK();
    }
    return launch_vl_and_flows(p, a, st);
  }
  return dense_combine_pass(s, p, a, st, pass);
}

constexpr int kDenseForwardPasses = 4;

template <int MODE>
int launch_adj(int N, const AdjSeq& q, dim3 grid, hipStream_t st) {
  if (N == 3) hipLaunchKernelGGL((k_adj<3, MODE>), grid, dim3(256), 0, st, q);
  else if (N == 2) hipLaunchKernelGGL((k_adj<2, MODE>), grid, dim3(256), 0, st, q);
  else hipLaunchKernelGGL((k_adj<1, MODE>), grid, dim3(256), 0, st, q);
  DENSE_CHECK();
  return EWS_OK;
}

// The adjoint of the combine and readout, given the forward's local terms / flows (loc, fl), chunk summaries and
// carries in the workspace: recomputes the prefix rows (the states), then LOCAL, CARRY and EMIT; leaves ds_t in loc
// and dM_t in fl.
// rows: the forward's prefix rows (W floats apart, the level-0 column first when the descriptor asks for it), or
// null. At d = 16 with the prefix readout they hold the states S_t in the padded layout, and the states pass is
// skipped.
int dense_adjoint(const ews_dense_desc* s, const DPlan& p, const Args& a, const float* grad_out, hipStream_t st,
                  const float* rows = nullptr) {
  const bool from_rows = rows && s->readout == EWS_READOUT_PREFIX && p.d == 16;
  if (!from_rows) {  // the forward's states S_t (padded rows)
    Seq q{};
    q.lv = a.loc; q.lv_bs = (long)p.n_int * p.LW; q.fl = a.fl; q.fl_bs = (long)p.n_int * 256;
    q.n = p.n_int; q.T = p.T; q.init = a.car; q.init_bs = (long)(p.C + 1) * p.LW;
    q.rows = a.pre; q.rows_bs = (long)p.n_int * p.LW; q.rows_ld = p.LW; q.padded = 1; q.lvl0 = 0; q.d = p.d;
    q.C = p.C;
    const int rc = launch_scan<false>(p.N, q, dim3(p.C, p.B), st);
    if (rc != EWS_OK) return rc;
  }
  const int ro = s->readout;
  if ((ro == EWS_READOUT_MEAN || ro == EWS_READOUT_MAX) && !s->level0) return EWS_ERR_OPTION;
  if (ro == EWS_READOUT_MAX) {  // per padded column (the level-0 column's cotangent goes nowhere)
    hipLaunchKernelGGL(k_argmax, dim3((p.LW + 255) / 256, p.B), dim3(256), 0, st, a.pre, p.n_int, p.LW, a.amax);
    DENSE_CHECK();
  }
  hipLaunchKernelGGL(k_lam_end, dim3((p.LW + 255) / 256, p.B), dim3(256), 0, st, a,
                     ro == EWS_READOUT_TERMINAL ? grad_out : nullptr, s->level0 ? 1 : 0);
  DENSE_CHECK();
  AdjSeq q{};
  q.n = p.n_int; q.T = p.T; q.C = p.C; q.d = p.d;
  q.gmode = ro == EWS_READOUT_PREFIX ? G_PREFIX : ro == EWS_READOUT_MEAN ? G_MEAN : ro == EWS_READOUT_MAX ? G_MAX
                                                                                                     : G_NONE;
  q.W = p.W; q.glvl0 = s->level0 ? 1 : 0; q.g = grad_out; q.amax = a.amax; q.gscale = 1.0f / (float)p.n_int;
  q.st = from_rows ? rows + (s->level0 ? 1 : 0) : a.pre;
  q.st_ld = from_rows ? p.W : p.LW;
  // LOCAL (the terminal readout has no in-chunk cotangents: the local parts are zero)
  if (q.gmode == G_NONE) {
    hipLaunchKernelGGL(k_zero_rows, dim3((p.LW + 255) / 256, p.B * p.C), dim3(256), 0, st, a.lloc, (long)p.LW,
                       p.B * p.C, p.LW);
    DENSE_CHECK();
  } else {
    AdjSeq ql = q;
    ql.lv = a.loc; ql.lv_bs = (long)p.n_int * p.LW; ql.fl = a.fl; ql.fl_bs = (long)p.n_int * 256;
    ql.lam = a.lloc;
    const int rc = launch_adj<ADJ_LOCAL>(p.N, ql, dim3(p.C, p.B), st);
    if (rc != EWS_OK) return rc;
  }
  {  // CARRY over the chunk summaries: Lambda_c = local_c + R(chunk c)^T Lambda_{c+1}, rows 1 .. C-1 of lam
    AdjSeq qc = q;
    qc.gmode = G_NONE;
    qc.lv = a.summ; qc.lv_bs = (long)p.C * p.LW; qc.fl = a.sfl; qc.fl_bs = (long)p.C * 256;
    qc.lloc = a.lloc; qc.lloc_bs = (long)p.C * p.LW;
    qc.n = p.C;
    if (p.NBc) {  // in the forward's blocks of kCarryBlock chunks, over its block summaries
      const int G = kCarryBlock, NB = p.NBc;
      AdjSeq q1 = qc;  // each block's local aggregate from a zero cotangent at its end
      q1.T = G; q1.init = nullptr; q1.lam = nullptr; q1.agg = a.bagg; q1.agg_bs = (long)NB * p.LW;
      int rc = launch_adj<ADJ_CARRY>(p.N, q1, dim3(NB, p.B), st);
      if (rc != EWS_OK) return rc;
      AdjSeq q2 = qc;  // the cotangent at every block end: over the block summaries from the terminal one
      q2.lv = a.bsumm; q2.lv_bs = (long)NB * p.LW; q2.fl = a.bsfl; q2.fl_bs = (long)NB * 256;
      q2.lloc = a.bagg; q2.lloc_bs = (long)NB * p.LW; q2.n = NB; q2.T = NB;
      q2.init = a.lam; q2.init_bs = (long)(p.C + 1) * p.LW; q2.init_off = p.C;
      q2.lam = a.bl; q2.lam_bs = (long)(NB + 1) * p.LW; q2.lam_lim = NB + 1;
      rc = launch_adj<ADJ_CARRY>(p.N, q2, dim3(1, p.B), st);
      if (rc != EWS_OK) return rc;
      AdjSeq q3 = qc;  // each block from the cotangent at its end: the chunk rows
      q3.T = G; q3.init = a.bl; q3.init_bs = (long)(NB + 1) * p.LW; q3.init_off = 1;
      q3.lam = a.lam; q3.lam_bs = (long)(p.C + 1) * p.LW; q3.lam_lim = p.C;
      rc = launch_adj<ADJ_CARRY>(p.N, q3, dim3(NB, p.B), st);
      if (rc != EWS_OK) return rc;
    } else {
      qc.T = p.C; qc.init = a.lam; qc.init_bs = (long)(p.C + 1) * p.LW; qc.init_off = p.C;
      qc.lam = a.lam; qc.lam_bs = (long)(p.C + 1) * p.LW; qc.lam_lim = p.C;
      const int rc = launch_adj<ADJ_CARRY>(p.N, qc, dim3(1, p.B), st);
      if (rc != EWS_OK) return rc;
    }
  }
  AdjSeq qe = q;
  qe.lv = a.loc; qe.lv_bs = (long)p.n_int * p.LW; qe.fl = a.fl; qe.fl_bs = (long)p.n_int * 256;
  qe.init = a.lam; qe.dlv = a.loc; qe.dfl = a.fl;
  return launch_adj<ADJ_EMIT>(p.N, qe, dim3(p.C, p.B), st);
}

}  // namespace

extern "C" {

size_t ews_dense_workspace_bytes(const ews_dense_desc* desc) {
  if (ews::wide::eligible(desc)) return ews::wide::workspace_bytes(desc, false);
  DPlan p;
  if (dense_plan(desc, p) != EWS_OK) return 0;
  return dense_ws(p, desc->readout).total;
}

int ews_dense_num_passes(void) { return kDenseForwardPasses; }

int ews_dense_forward_pass(const ews_dense_desc* desc, int pass, const float* path, const float* clock,
                           const float* A, float* out, void* workspace, ews_stream_t stream) {
  DPlan p;
  const int rc = dense_plan(desc, p);
  if (rc != EWS_OK) return rc;
  if (!path || !clock || !A || !out || !workspace) return EWS_ERR_NULL;
  if (pass < 0 || pass >= kDenseForwardPasses) return EWS_ERR_OPTION;
  const Args a = dense_args(desc, p, path, clock, A, out, workspace);
  return dense_forward_pass(desc, p, a, (hipStream_t)stream, pass);
}

int ews_dense_forward(const ews_dense_desc* desc, const float* path, const float* clock, const float* A,
                      float* out, void* workspace, ews_stream_t stream) {
  if (ews::wide::eligible(desc))
    return ews::wide::forward(desc, path, clock, A, out, workspace, false, (hipStream_t)stream);
  for (int pass = 0; pass < kDenseForwardPasses; ++pass) {
    const int rc = ews_dense_forward_pass(desc, pass, path, clock, A, out, workspace, stream);
    if (rc != EWS_OK) return rc;
  }
  return EWS_OK;
}

int ews_dense_forward_keep(const ews_dense_desc* desc, const float* path, const float* clock, const float* A,
                           float* out, void* workspace, ews_stream_t stream) {
  // d > 16: the forward runs in the backward's workspace, and ews_dense_backward_kept starts from what it left
  if (ews::wide::eligible(desc))
    return ews::wide::forward(desc, path, clock, A, out, workspace, true, (hipStream_t)stream);
  DPlan p;
  const int rc = dense_plan(desc, p);
  if (rc != EWS_OK) return rc;
  if (!path || !clock || !A || !out || !workspace) return EWS_ERR_NULL;
  const Args a = dense_args(desc, p, path, clock, A, out, workspace, true);  // the backward's layout
  for (int pass = 0; pass < kDenseForwardPasses; ++pass) {
    const int r = dense_forward_pass(desc, p, a, (hipStream_t)stream, pass);
    if (r != EWS_OK) return r;
  }
  return EWS_OK;
}

int ews_dense_local_terms(const ews_dense_desc* desc, const float* path, const float* clock, const float* A,
                          float* levels, float* flows, void* workspace, ews_stream_t stream) {
  DPlan p;
  const int rc = dense_plan(desc, p);
  if (rc != EWS_OK) return rc;
  if (!path || !clock || !A || !levels || !flows || !workspace) return EWS_ERR_NULL;
  ews_dense_desc s = *desc;
  s.level0 = 0;
  DPlan q = p;
  q.W = p.D;
  const Args a = dense_args(&s, q, path, clock, A, nullptr, workspace);
  hipStream_t st = (hipStream_t)stream;
  const int r0 = dense_forward_pass(&s, q, a, st, 0);
  if (r0 != EWS_OK) return r0;
  hipLaunchKernelGGL(k_unpad_outputs, dim3(p.B * p.n_int), dim3(256), 0, st, a, levels, flows);
  DENSE_CHECK();
  return EWS_OK;
}

size_t ews_dense_backward_workspace_bytes(const ews_dense_desc* desc) {
  if (ews::wide::eligible(desc)) return ews::wide::workspace_bytes(desc, true);
  DPlan p;
  if (dense_plan(desc, p) != EWS_OK) return 0;
  return dense_ws(p, desc->readout, true).total;
}

int ews_dense_combine_backward(const ews_dense_desc* desc, const float* levels, const float* flows,
                               const float* grad_out, float* grad_levels, float* grad_flows, void* workspace,
                               ews_stream_t stream) {
  DPlan p;
  const int rc = dense_plan(desc, p);
  if (rc != EWS_OK) return rc;
  if (!levels || !flows || !grad_out || !grad_levels || !grad_flows || !workspace) return EWS_ERR_NULL;
  const Args a = dense_args(desc, p, nullptr, nullptr, nullptr, nullptr, workspace, true);
  hipStream_t st = (hipStream_t)stream;
  hipLaunchKernelGGL(k_pad_inputs, dim3(p.B * p.n_int), dim3(256), 0, st, a, levels, flows);
  DENSE_CHECK();
  for (int pass = 1; pass <= 2; ++pass) {
    const int r = dense_combine_pass(desc, p, a, st, pass);
    if (r != EWS_OK) return r;
  }
  const int r = dense_adjoint(desc, p, a, grad_out, st);
  if (r != EWS_OK) return r;
  Args u = a;
  u.W = p.D + u.lvl0;  // k_unpad_outputs writes levels with the packed width D = W - lvl0
  hipLaunchKernelGGL(k_unpad_outputs, dim3(p.B * p.n_int), dim3(256), 0, st, u, grad_levels, grad_flows);
  DENSE_CHECK();
  return EWS_OK;
}

}  // extern "C"

namespace {
// The leaf's and the flows' adjoints per interval, given ds_t in loc and dM_t in fl: path, clock and A gradients.
int dense_leaf_adjoint(const ews_dense_desc* desc, const DPlan& p, const Args& a, void* workspace, float* grad_path,
                       float* grad_clock, float* grad_A, hipStream_t st) {
  const DWs w = dense_ws(p, desc->readout, true);
  char* ws = (char*)workspace;
  LeafBwd o;
  o.dv = (float*)(ws + w.dv); o.dh = (float*)(ws + w.dh); o.dsh = (float*)(ws + w.dsh); o.part = (float*)(ws + w.part);
  o.dshi = (float*)(ws + w.dshi);
  double* hsum = (double*)(ws + w.hsum);
  const long total = (long)p.B * p.n_int;
  const int grid = (int)(total < kLeafBwdBlocks ? total : kLeafBwdBlocks);
  const size_t lshm = p.leaf == EWS_LEAF_VAN_LOAN ? 0 : (size_t)6 * (p.q + 1) * 16 * 4;  // k_leaf_bwd's letters
  const bool bs = p.leaf == EWS_LEAF_BLOCK_SERIES;
  float* bsdv = (float*)(ws + w.bsdv);
  float* bsdh = (float*)(ws + w.bsdh);
  float* bspart = (float*)(ws + w.bspart);
  if (bs) {  // the exact level 1's adjoint first: it takes the level-1 cotangent out of loc
    hipLaunchKernelGGL(k_bs_level1_bwd, dim3(grid), dim3(256), 0, st, a, bsdv, bsdh, bspart);
    DENSE_CHECK();
  }
#define EWS_LEAF_BWD(KER, NN)                                                                               \
  do {                                                                                                      \
    if (p.chen_expm == EWS_EXPM_EXACT) hipLaunchKernelGGL((KER<NN, true>), dim3(grid), dim3(256), lshm, st, a, o); \
    else hipLaunchKernelGGL((KER<NN, false>), dim3(grid), dim3(256), lshm, st, a, o);                        \
  } while (0)
  if (p.leaf == EWS_LEAF_VAN_LOAN) {
    if (p.N == 1) EWS_LEAF_BWD(k_vl_bwd, 1);
    else if (p.N == 2) EWS_LEAF_BWD(k_vl_bwd, 2);
    else EWS_LEAF_BWD(k_vl_bwd, 3);
  } else {
    if (p.N == 1) EWS_LEAF_BWD(k_leaf_bwd, 1);
    else if (p.N == 2) EWS_LEAF_BWD(k_leaf_bwd, 2);
    else EWS_LEAF_BWD(k_leaf_bwd, 3);
  }
#undef EWS_LEAF_BWD
  DENSE_CHECK();
  if (bs) {
    hipLaunchKernelGGL(k_bs_add, dim3(256), dim3(256), 0, st, a, o, bsdv, bsdh);
    DENSE_CHECK();
  }
  hipLaunchKernelGGL(k_part_reduce, dim3(HP + 1, PRS), dim3(256), 0, st, o.part, grid, hsum);
  DENSE_CHECK();
  hipLaunchKernelGGL(k_dA, dim3(1), dim3(256), 0, st, a, hsum, grad_A);
  DENSE_CHECK();
  if (bs) {
    hipLaunchKernelGGL(k_bs_dA, dim3(1), dim3(256), 0, st, a, bspart, grid, grad_A);
    DENSE_CHECK();
  }
  hipLaunchKernelGGL(k_dsh_reduce, dim3(p.B), dim3(256), 0, st, a, o);
  DENSE_CHECK();
  hipLaunchKernelGGL(k_knots, dim3((p.L + 255) / 256, p.B), dim3(256), 0, st, a, o, grad_path, grad_clock);
  DENSE_CHECK();
  return EWS_OK;
}
}  // namespace

extern "C" {

int ews_dense_backward(const ews_dense_desc* desc, const float* path, const float* clock, const float* A,
                       const float* grad_out, float* grad_path, float* grad_clock, float* grad_A, void* workspace,
                       ews_stream_t stream) {
  if (ews::wide::eligible(desc))
    return ews::wide::backward(desc, path, clock, A, grad_out, grad_path, grad_clock, grad_A, workspace, false,
                               (hipStream_t)stream);
  DPlan p;
  const int rc = dense_plan(desc, p);
  if (rc != EWS_OK) return rc;
  if (!path || !clock || !A || !grad_out || !grad_path || !grad_A || !workspace) return EWS_ERR_NULL;
  const Args a = dense_args(desc, p, path, clock, A, nullptr, workspace, true);
  hipStream_t st = (hipStream_t)stream;
  for (int pass = 0; pass <= 2; ++pass) {  // the forward up to the carries
    const int r = dense_forward_pass(desc, p, a, st, pass);
    if (r != EWS_OK) return r;
  }
  const int r = dense_adjoint(desc, p, a, grad_out, st);
  if (r != EWS_OK) return r;
  return dense_leaf_adjoint(desc, p, a, workspace, grad_path, grad_clock, grad_A, st);
}

int ews_dense_backward_kept(const ews_dense_desc* desc, const float* path, const float* clock, const float* A,
                            const float* out, const float* grad_out, float* grad_path, float* grad_clock,
                            float* grad_A, void* workspace, ews_stream_t stream) {
  if (ews::wide::eligible(desc))
    return ews::wide::backward(desc, path, clock, A, grad_out, grad_path, grad_clock, grad_A, workspace, true,
                               (hipStream_t)stream);
  DPlan p;
  const int rc = dense_plan(desc, p);
  if (rc != EWS_OK) return rc;
  if (!path || !clock || !A || !grad_out || !grad_path || !grad_A || !workspace) return EWS_ERR_NULL;
  const Args a = dense_args(desc, p, path, clock, A, nullptr, workspace, true);
  hipStream_t st = (hipStream_t)stream;
  // the leaf, flows, summaries and carries are kept; the states come from the forward's rows when given
  const int r = dense_adjoint(desc, p, a, grad_out, st, out);
  if (r != EWS_OK) return r;
  return dense_leaf_adjoint(desc, p, a, workspace, grad_path, grad_clock, grad_A, st);
}

int ews_dense_combine(const ews_dense_desc* desc, const float* levels, const float* flows, float* out,
                      void* workspace, ews_stream_t stream) {
  DPlan p;
  const int rc = dense_plan(desc, p);
  if (rc != EWS_OK) return rc;
  if (!levels || !flows || !out || !workspace) return EWS_ERR_NULL;
  Args a = dense_args(desc, p, nullptr, nullptr, nullptr, out, workspace);
  hipStream_t st = (hipStream_t)stream;
  // k_pad_inputs reads levels with the packed width D = W - lvl0
  hipLaunchKernelGGL(k_pad_inputs, dim3(p.B * p.n_int), dim3(256), 0, st, a, levels, flows);
  DENSE_CHECK();
  for (int pass = 1; pass < kDenseForwardPasses; ++pass) {
    const int r = dense_combine_pass(desc, p, a, st, pass);
    if (r != EWS_OK) return r;
  }
  return EWS_OK;
}

size_t ews_token_scan_workspace_bytes(const ews_dense_desc* desc, int vocab) {
  DPlan p;
  if (vocab < 1 || dense_plan(desc, p) != EWS_OK) return 0;
  const size_t f = dense_ws(p, desc->readout, false).total, b = dense_ws(p, desc->readout, true).total;
  const size_t nch = ((size_t)p.B * p.n_int + kTokChunk - 1) / kTokChunk;
  const size_t part = al256(nch * (size_t)vocab * (p.LW + 256) * 4);
  return (f > b + part ? f : b + part);
}

int ews_token_scan(const ews_dense_desc* desc, const int32_t* token_ids, const uint8_t* mask, const float* P_cache,
                   const float* D_cache, int vocab, float* out, void* workspace, ews_stream_t stream) {
  DPlan p;
  const int rc = dense_plan(desc, p);
  if (rc != EWS_OK) return rc;
  if (vocab < 1) return EWS_ERR_SHAPE;
  if (!token_ids || !P_cache || !D_cache || !out || !workspace) return EWS_ERR_NULL;
  Args a = dense_args(desc, p, nullptr, nullptr, nullptr, out, workspace);
  hipStream_t st = (hipStream_t)stream;
  hipLaunchKernelGGL(k_pad_tokens, dim3((p.B * p.n_int + 3) / 4), dim3(256), 0, st, a, token_ids, mask, P_cache, D_cache,
                     vocab, p.D);
  DENSE_CHECK();
  for (int pass = 1; pass < kDenseForwardPasses; ++pass) {
    const int r = dense_combine_pass(desc, p, a, st, pass);
    if (r != EWS_OK) return r;
  }
  return EWS_OK;
}

int ews_token_scan_backward(const ews_dense_desc* desc, const int32_t* token_ids, const uint8_t* mask,
                            const float* P_cache, const float* D_cache, int vocab, const float* grad_out,
                            float* grad_P_cache, float* grad_D_cache, void* workspace, ews_stream_t stream) {
  DPlan p;
  const int rc = dense_plan(desc, p);
  if (rc != EWS_OK) return rc;
  if (vocab < 1) return EWS_ERR_SHAPE;
  if (!token_ids || !P_cache || !D_cache || !grad_out || !grad_P_cache || !grad_D_cache || !workspace)
    return EWS_ERR_NULL;
  const Args a = dense_args(desc, p, nullptr, nullptr, nullptr, nullptr, workspace, true);
  hipStream_t st = (hipStream_t)stream;
  hipLaunchKernelGGL(k_pad_tokens, dim3((p.B * p.n_int + 3) / 4), dim3(256), 0, st, a, token_ids, mask, P_cache, D_cache,
                     vocab, p.D);
  DENSE_CHECK();
  for (int pass = 1; pass <= 2; ++pass) {
    const int r = dense_combine_pass(desc, p, a, st, pass);
    if (r != EWS_OK) return r;
  }
  const int r = dense_adjoint(desc, p, a, grad_out, st);
  if (r != EWS_OK) return r;
  float* part = (float*)((char*)workspace + dense_ws(p, desc->readout, true).total);
  const int nch = (int)(((long)p.B * p.n_int + kTokChunk - 1) / kTokChunk);
  const int E = p.LW + 256;
  hipLaunchKernelGGL(k_token_grads1, dim3((E + 255) / 256, nch, (vocab + 15) / 16), dim3(256), 0, st, a, token_ids,
                     mask, vocab, part);
  DENSE_CHECK();
  hipLaunchKernelGGL(k_token_grads2, dim3((int)(((long)vocab * E + 63) / 64)), dim3(256), 0, st, a, part, nch,
                     vocab, p.D, grad_P_cache, grad_D_cache);
  DENSE_CHECK();
  return EWS_OK;
}

int ews_dense_local_terms_backward(const ews_dense_desc* desc, const float* path, const float* clock, const float* A,
                                   const float* grad_levels, const float* grad_flows, float* grad_path,
                                   float* grad_clock, float* grad_A, void* workspace, ews_stream_t stream) {
  DPlan p;
  const int rc = dense_plan(desc, p);
  if (rc != EWS_OK) return rc;
  if (!path || !clock || !A || !grad_levels || !grad_flows || !grad_path || !grad_A || !workspace)
    return EWS_ERR_NULL;
  const Args a = dense_args(desc, p, path, clock, A, nullptr, workspace, true);
  hipStream_t st = (hipStream_t)stream;
  const int r = dense_forward_pass(desc, p, a, st, 0);  // the leaf's recompute state (powers, Van Loan saves)
  if (r != EWS_OK) return r;
  Args u = a;
  u.W = p.D + u.lvl0;  // k_pad_inputs reads levels with the packed width D = W - lvl0
  hipLaunchKernelGGL(k_pad_inputs, dim3(p.B * p.n_int), dim3(256), 0, st, u, grad_levels, grad_flows);
  DENSE_CHECK();
  return dense_leaf_adjoint(desc, p, a, workspace, grad_path, grad_clock, grad_A, st);
}

}  // extern "C"
