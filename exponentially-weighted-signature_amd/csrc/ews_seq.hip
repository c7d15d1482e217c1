// Per-sample sequential EWS scan for real diagonal generators (d <= 32), depth 2, prefix readouts: one workgroup
// per sample, one lane per level-2 pair (j, k), the whole sequence walked step by step. There is no chunk scan and
// no carry between workgroups, so it suits many samples of moderate length (one block of the stacked LogEWS
// configuration: B = 256 sequences of 512 steps at d = 32), where the chunk kernels need one 1,024-lane workgroup
// per 16-step chunk and recompute every chunk's states from checkpoints.
//
// Math (reference sign, real diagonal A = diag(lambda), node x = -h lambda): per step, with c_j = rho_j S1_j,
//     S2[j,k] <- L_jk S2[j,k] + c_j phi_k v_k + D_jk v_j v_k,     S1_j <- c_j + phi_j v_j
// rho = e^x, phi = exp[0, x], L_jk = e^{x_j + x_k}, D_jk = exp[0, x_j, x_j + x_k]: the closed forms of
// ews/core/kernels/plane_engine.py:134-152 on 1x1 blocks, or their order-q truncations for the series leaves
// (node1q / dd3q). Each lane carries its pair and the level-1 states of its row j and column k, computed by the
// same operations as the row's own lanes (so bit for bit equal), and the forward step needs no lane exchange.
//
// Readouts: the flat prefix rows (level 0, level 1, level 2 row-major; ews/core/output_format.py:12-37) or the
// compressed log rows of LogEWS at depth 2 (ews/layer.py:488-517 with signax's signature_to_logsignature): level 1,
// then S2[j,k] - S1_j S1_k / 2 at the Lyndon words j < k in lexicographic order, written straight from the scan.
//
// Backward (the reference's VJP, ews/core/kernels/pallas_combine.py:1698-1798, restated for one sequential pass):
// the forward leaves a checkpoint of the state every 16 steps; block by block from the end, the block's states are
// recomputed into registers (the same operations, so the same bits) and the adjoint steps back through them:
//     Lam2 = lam2 + g2, Lam1 = lam1 + g1,  gc_j = Lam1_j + sum_k Lam2[j,k] phi_k v_k   (a 32-lane row sum)
//     lam1_j <- rho_j gc_j,    lam2 <- L Lam2
//     dv_m = phi_m Lam1_m + sum_k Lam2[m,k] D_mk v_k + sum_j Lam2[j,m] (phi_m c_j + D_jm v_j)
// g1 of a log row adds -1/2 sum_{k != j} g[min(j,k), max(j,k)] S1_k (the log's level-2 term). The column sums of
// dv go through LDS, 8 steps at a time, off the sequential chain; the cotangent rows arrive in LDS by asynchronous
// copies (global_load_lds) issued 8 steps ahead. Parameter gradients collect h times each coefficient's cotangent
// times its node derivative (a coefficient c(x), x = -h lambda, gives -h c'(x)).
//
// Per-step coefficients: one set when every clock step of the sample equals the mean step; first-order models in
// the step around the mean when every step is within 2^-16 / (2 max lambda) of it (a uniform clock in float32, the
// chunk kernels' test); otherwise each step's coefficients are evaluated exactly.
#include <hip/hip_runtime.h>

#include "ews_args.h"
#include "ews_hip.h"
#include "ews_numerics.h"
#include "ews_seq.h"

namespace ews {
namespace seq {

constexpr int CB = kSeqCB;
constexpr int MAXK = kSeqMaxK;
constexpr int RS = 32;                // lanes per pair row: lane = 32 j + k
constexpr int Q = 8;                  // steps of column partials staged before their reduction
constexpr int MAXW = MAXK * RS / 64;  // wavefronts per workgroup at d = 32
static_assert(CB <= RS, "one staged increment per lane");

// DPP row rotation inside rows of 16 lanes (update_dpp with a zero old value folds into the add as v_add_f32_dpp)
#define EWS_SEQ_ROR(v, n) __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x120 + (n), 0xf, 0xf, true))
// value of lane l ^ 16 added to lane l's: v_permlane16_swap exchanges the odd 16-lane rows of one copy with the even
// rows of the other, so the two results hold each lane's and its partner's value (a VALU op, no LDS round trip)
__device__ __forceinline__ float add_xor16(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
// sum over the 32 lanes of a pair row, in every lane of the row
__device__ __forceinline__ float row_sum(float v) {
  v += EWS_SEQ_ROR(v, 8);
  v += EWS_SEQ_ROR(v, 4);
  v += EWS_SEQ_ROR(v, 2);
  v += EWS_SEQ_ROR(v, 1);
  return add_xor16(v);
}

// Coefficients of the lane's pair (j, k) at one clock step.
struct Co {
  float rj, rk, pj, pk, L, D;
};
// Their derivatives in the nodes: rho' = rho, phi' = exp[0, x, x], L' = L (in x_j + x_k), and for D(x_j, x_j + x_k)
// the x_j derivative Dx + Dy and the x_k derivative Dy.
struct Nd {
  float rj, pj, pk, L, Dxy, Dy;
};

// c: coefficients at step h; dh: their derivatives in h; nd: node derivatives
__device__ __forceinline__ void eval_co(const DiagArgs& a, float lj, float lk, float h, Co& c, Co& dh, Nd& nd) {
  const float uj = -lj, uk = -lk, ub = uj + uk;
  const Node1<float> nj = node1q(h * uj, a.sq1), nk = node1q(h * uk, a.sq1);
  const DD3<float> dd = dd3q<float, true>(h * uj, h * ub, a.sq2);
  c = Co{nj.e, nk.e, nj.p, nk.p, expv(h * ub), dd.d};
  nd = Nd{nj.e, nj.dp, nk.dp, c.L, dd.dx + dd.dy, dd.dy};
  dh = Co{uj * nj.e, uk * nk.e, uj * nj.dp, uk * nk.dp, ub * c.L, dd.dx * uj + dd.dy * ub};
}
__device__ __forceinline__ Co lin(const Co& c0, const Co& c1, float dl) {
  return Co{fmaf(c1.rj, dl, c0.rj), fmaf(c1.rk, dl, c0.rk), fmaf(c1.pj, dl, c0.pj), fmaf(c1.pk, dl, c0.pk),
            fmaf(c1.L, dl, c0.L), fmaf(c1.D, dl, c0.D)};
}

// The sample's clock model: the mean step, and how the per-step coefficients are formed: every step equal to the
// mean (one set of coefficients), every step within 2^-16 / (2 max lambda) of it (first-order models in the step,
// the chunk kernels' test over the whole sample), or exact coefficients at every step.
enum { CK_UNIFORM = 0, CK_LINEAR = 1, CK_EXACT = 2 };
struct Clock {
  float hbar;
  int mode;
};
__device__ Clock sample_clock(const DiagArgs& a, int b, float* s_red) {
  const float* th = a.clock + (size_t)b * a.L;
  const int n = a.n_int, tid = threadIdx.x;
  Clock ck;
  ck.hbar = (th[n] - th[0]) / (float)n;
  float dev = isfinite(ck.hbar) ? 0.0f : INFINITY;
  for (int t = tid; t < n; t += blockDim.x) {
    const float dl = fabsf((th[t + 1] - th[t]) - ck.hbar);
    dev = dl <= 3.0e38f ? fmaxf(dev, dl) : INFINITY;  // a NaN or infinite step fails the test
  }
  for (int o = 32; o > 0; o >>= 1) dev = fmaxf(dev, __shfl_xor(dev, o, 64));
  if ((tid & 63) == 0) s_red[tid >> 6] = dev;
  float R = 0.0f;
  for (int m = 0; m < a.K; ++m) R = fmaxf(R, fabsf(a.params[m]));
  __syncthreads();
  float mx = 0.0f;
  for (int w = 0; w < (int)(blockDim.x >> 6); ++w) mx = fmaxf(mx, s_red[w]);
  __syncthreads();
  ck.mode = mx == 0.0f ? CK_UNIFORM : (mx * 2.0f * R < 1.52587890625e-5f ? CK_LINEAR : CK_EXACT);  // 2^-16
  return ck;
}

// The lane's coefficients at the mean step (value and step derivative), and their evaluation at a step h under the
// clock mode (node derivatives only in the exact mode: the others apply them once, at the end).
struct Model {
  Co c0, c1;
  float hbar;
};
template <int MODE>
__device__ __forceinline__ void coef_at(const DiagArgs& a, const Model& md, float lj, float lk, float h, Co& c,
                                        Co& cd, Nd& cn) {
  if constexpr (MODE == CK_UNIFORM) {
    c = md.c0;
    cd = md.c1;
  } else if constexpr (MODE == CK_LINEAR) {
    c = lin(md.c0, md.c1, h - md.hbar);
    cd = md.c1;
  } else {
    eval_co(a, lj, lk, h, c, cd, cn);
  }
}

__device__ __forceinline__ float path_at(const DiagArgs& a, size_t idx) {
  if (a.path_bf16) return __uint_as_float(((unsigned)reinterpret_cast<const unsigned short*>(a.path)[idx]) << 16);
  return reinterpret_cast<const float*>(a.path)[idx];
}

// One block's increments v[s][m] (CB x K, one per lane) and clock steps h[s]: loaded into registers ahead of use
// (the next block's while the current one runs), then written to LDS.
struct Stage {
  float v, h;
};
__device__ __forceinline__ void stage_load(const DiagArgs& a, int b, int blk, Stage& st) {
  const int ns = min(CB, a.n_int - blk * CB), K = a.K, e = threadIdx.x;
  const int s = e / K, m = e - s * K;
  const size_t t0 = (size_t)b * a.L + (size_t)blk * CB;
  st.v = s < ns ? path_at(a, (t0 + s + 1) * a.d + m) - path_at(a, (t0 + s) * a.d + m) : 0.0f;
  st.h = e < ns ? a.clock[t0 + e + 1] - a.clock[t0 + e] : 0.0f;
}
__device__ __forceinline__ void stage_store(const DiagArgs& a, const Stage& st, float* s_v, float* s_h) {
  const int e = threadIdx.x;
  if (e < CB * a.K) s_v[e] = st.v;
  if (e < CB) s_h[e] = st.h;
}

// index of the Lyndon word (j, k), j < k, among the words of length 2 in lexicographic order
__device__ __forceinline__ int witt2(int j, int k, int K) { return j * (2 * K - j - 1) / 2 + k - j - 1; }

// One forward step of the lane's states (identical operations in the forward, the checkpoints and the backward's
// recomputation).
__device__ __forceinline__ void fstep(const Co& c, float vj, float vk, float& S1j, float& S1k, float& S2) {
  const float cj = c.rj * S1j;
  S2 = fmaf(c.L, S2, fmaf(cj, c.pk * vk, c.D * (vj * vk)));
  S1j = fmaf(c.pj, vj, cj);
  S1k = fmaf(c.pk, vk, c.rk * S1k);
}

// value of lane l ^ 32 added to lane l's (v_permlane32_swap exchanges the wavefront's two halves)
__device__ __forceinline__ float add_xor32(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Workgroup barrier ordering LDS only: global loads issued before it (prefetches) stay in flight.
__device__ __forceinline__ void lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}
// Asynchronous copy of n contiguous floats into LDS (global_load_lds: each lane's dword lands at the wavefront's
// LDS base + 4 x lane), and the barrier after which every wavefront's copies have landed.
typedef __attribute__((address_space(3))) void lds_void_t;
__device__ __forceinline__ void lds_dma(float* dst, const float* src, int n) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, nw = blockDim.x >> 6;
  for (int base = w * 64; base < n; base += nw * 64) {
    const int idx = base + lane;
    if (idx < n) __builtin_amdgcn_global_load_lds((const void*)(src + idx), (lds_void_t*)(dst + base), 4, 0, 0);
  }
}
__device__ __forceinline__ void dma_sync() {
  __builtin_amdgcn_s_waitcnt(0);
  lds_sync();
}

// ------------------------------------------------------------------------------------------------ forward
struct FwdLds {
  float v[2][CB * MAXK], h[2][CB], red[MAXW];
};

// KC: the width as a compile-time constant (32: every lane active), 0 otherwise. A log row is written by the lanes
// j <= k, one element each: level 1 by the diagonal lanes, the Lyndon coefficient (j, k) by the others.
template <bool LOG, int MODE, int KC>
__device__ __forceinline__ void fwd_body(const DiagArgs& a, FwdLds& sm, const Model& md, float lj, float lk) {
  const int b = blockIdx.x, p = threadIdx.x, j = p / RS, k = p % RS, n = a.n_int, NT = blockDim.x;
  const int K = KC ? KC : a.K;
  const int W = (KC && LOG) ? KC + KC * (KC - 1) / 2 : a.W;
  const bool act = KC ? true : (j < K && k < K);
  const int jj = act ? j : 0, kk = act ? k : 0;
  const bool wr = LOG ? (act && j <= k) : act;  // the lane writes one element of every row
  const int off = LOG ? (j == k ? jj : K + witt2(jj, kk, K)) : a.off2 + jj * K + kk;
  const bool wr1 = !LOG && j == 0 && act;        // flat rows: level 1 from the first pair row
  float S1j = 0.0f, S1k = 0.0f, S2 = 0.0f;
  const int nb = seq_blocks(n);
  float* ckp = a.seqck ? a.seqck + (size_t)b * seq_ckpt_floats(K, n) : nullptr;
  Co cu{};
  if constexpr (MODE == CK_UNIFORM) cu = md.c0;
  Stage st;
  stage_load(a, b, 0, st);
  stage_store(a, st, sm.v[0], sm.h[0]);
  __syncthreads();
  for (int blk = 0; blk < nb; ++blk) {
    if (ckp) {
      float* cpt = ckp + (size_t)blk * (NT + K);
      cpt[p] = S2;
      if (j == 0 && act) cpt[NT + k] = S1k;
    }
    if (blk + 1 < nb) stage_load(a, b, blk + 1, st);
    const float* sv = sm.v[blk & 1];
    const float* sh = sm.h[blk & 1];
    const int ns = min(CB, n - blk * CB);
    float* row = a.out + ((size_t)b * n + (size_t)blk * CB) * W;
    auto step = [&](int s) {
      Co c, cd;
      Nd cn;
      if constexpr (MODE == CK_UNIFORM) c = cu;
      else coef_at<MODE>(a, md, lj, lk, sh[s], c, cd, cn);
      const float vj = act ? sv[s * K + jj] : 0.0f;
      const float vk = act ? sv[s * K + kk] : 0.0f;
      fstep(c, vj, vk, S1j, S1k, S2);
      float* r = row + (size_t)s * W;
      if constexpr (!LOG) {
        if (wr) r[off] = S2;
        if (wr1) r[a.off1 + k] = S1k;
        if (a.lvl0 && p == 0) r[0] = 1.0f;
      } else {
        if (wr) r[off] = j == k ? S1k : fmaf(-0.5f * S1j, S1k, S2);
      }
    };
    if constexpr (LOG && KC) {  // fixed row length: the unrolled steps store at immediate offsets
#pragma unroll
      for (int s = 0; s < CB; ++s)
        if (s < ns) step(s);
    } else {
      for (int s = 0; s < ns; ++s) step(s);
    }
    if (blk + 1 < nb) stage_store(a, st, sm.v[(blk + 1) & 1], sm.h[(blk + 1) & 1]);
    lds_sync();  // the checkpoint and row stores need no ordering here
  }
}

template <bool LOG, int KC>
__global__ __launch_bounds__(1024) void k_seq_fwd(DiagArgs a) {
  __shared__ FwdLds sm;
  const int p = threadIdx.x, j = p / RS, k = p % RS;
  const bool act = j < a.K && k < a.K;
  const float lj = act ? a.params[j] : 0.0f, lk = act ? a.params[k] : 0.0f;
  const Clock ck = sample_clock(a, blockIdx.x, sm.red);
  Model md{};
  md.hbar = ck.hbar;
  Nd nd;
  if (ck.mode != CK_EXACT) eval_co(a, lj, lk, ck.hbar, md.c0, md.c1, nd);
  if (ck.mode == CK_UNIFORM) fwd_body<LOG, CK_UNIFORM, KC>(a, sm, md, lj, lk);
  else if (ck.mode == CK_LINEAR) fwd_body<LOG, CK_LINEAR, KC>(a, sm, md, lj, lk);
  else fwd_body<LOG, CK_EXACT, KC>(a, sm, md, lj, lk);
}

// ------------------------------------------------------------------------------------------------ backward
struct BwdLds {
  float v[CB * MAXK], h[CB], red[MAXW];
  float s1[CB + 1][MAXK];          // level 1 before step s of the block (row s); row ns: after the block
  float col[CB][MAXW][RS];         // column parts of dv: per wavefront, its two rows summed
  float rowp[CB][MAXK];            // row parts of dv
  float dhw[CB][MAXW];             // clock-step cotangent per wavefront
  float dv[CB][MAXK], dh[CB];      // dv / dh of the block's steps
  float next[2][MAXK], nexth[2];   // dv / dh of the step after the block (0 after the last), by block parity
  float gcol[MAXK][RS], grow[MAXK];
};

// Cotangent rows are staged Q steps at a time into two LDS buffers of Q x W floats (dynamic LDS), copied
// asynchronously one group ahead of their use.
//
// The adjoint step in the form the lanes evaluate it, with t_jk = Lam2 phi_k v_k and two row sums per step:
//     X_j = sum_k (t_jk - G_jk S1_k / 2)  (log rows; X_j = sum_k t_jk for flat rows),  gc_j = lam1_j + g1_j + X_j
//     Y_j = sum_k Lam2 (D_jk - phi_j phi_k) v_k,   dv_j (row part) = phi_j gc_j + Y_j
// (Lam1 = gc - sum_k t_jk, so phi_j Lam1 + sum_k Lam2 D v_k = phi_j gc + Y). The phi_j cotangent h Lam1 v_j is
// collected as h gc v_j (the same in every lane of the row) minus h t_jk v_j per lane, row-summed once at the end.
// KC: the width as a compile-time constant (32: every lane active, fixed row length of the log rows), 0 otherwise.
template <bool LOG, bool DH, int MODE, int KC>
__device__ __forceinline__ void bwd_body(const DiagArgs& a, BwdLds& sm, float* sg, const Model& md, float lj,
                                         float lk) {
  const int b = blockIdx.x, p = threadIdx.x, j = p / RS, k = p % RS, n = a.n_int, NT = blockDim.x;
  const int K = KC ? KC : a.K;
  const int W = (KC && LOG) ? KC + KC * (KC - 1) / 2 : a.W;
  const int w = p >> 6, nw = NT >> 6;
  const bool act = KC ? true : (j < K && k < K);
  const bool rowl = KC ? true : j < K;  // a lane of a real pair row
  const int nb = seq_blocks(n);
  constexpr int NG = CB / Q;  // groups per block
  static_assert(CB % Q == 0 && NG % 2 == 0, "group g of every block stages into buffer g & 1");
  const float* ckp = a.seqck + (size_t)b * seq_ckpt_floats(K, n);
  const float* gsm = a.gout + (size_t)b * n * W;
  auto dma_group = [&](int blk, int g) {
    const int rows = min(Q, min(CB, n - blk * CB) - g * Q);
    if (rows > 0) lds_dma(sg + (g & 1) * Q * W, gsm + (size_t)(blk * CB + g * Q) * W, rows * W);
  };
  // lane constants: where the lane's cotangents sit in a staged row, and 0/1 masks
  const int jj = act ? j : 0, kk = act ? k : 0;
  const int off_g2 = LOG ? (jj == kk ? 0 : K + witt2(min(jj, kk), max(jj, kk), K)) : a.off2 + jj * K + kk;
  const int off_g1 = LOG ? jj : a.off1 + jj;
  // log rows: G' = -G/2 for the lanes j != k (the level-1 term of the log) and g2 = -2 G' for j < k
  const float m_g = (act && (!LOG || j != k)) ? (LOG ? -0.5f : 1.0f) : 0.0f;
  const float m_u = (act && (!LOG || j < k)) ? (LOG ? -2.0f : 1.0f) : 0.0f;
  const float m_row = rowl ? 1.0f : 0.0f;
  const float m_act = act ? 1.0f : 0.0f;
  const float m_k0 = (k == 0 && rowl) ? 1.0f : 0.0f;
  if (p < MAXK) sm.next[(nb - 1 + 1) & 1][p] = 0.0f;
  if (p == 0) sm.nexth[(nb - 1 + 1) & 1] = 0.0f;
  // the level-1 rows past the last channel stay zero (read by the padded lanes of narrow widths)
  for (int e = p; e < (CB + 1) * MAXK; e += NT) (&sm.s1[0][0])[e] = 0.0f;
  // prologue: the last block's inputs, checkpoint and last cotangent group
  Stage st;
  stage_load(a, b, nb - 1, st);
  float ck2 = ckp[(size_t)(nb - 1) * (NT + K) + p];
  float ck1 = rowl ? ckp[(size_t)(nb - 1) * (NT + K) + NT + j] : 0.0f;
  dma_group(nb - 1, NG - 1);
  float lam1 = 0.0f, lam2 = 0.0f;  // cotangents of S1_j (replicated along the row) and of the lane's S2
  // parameter cotangents (see above; the exact mode folds each step's node derivative in, the model modes apply the
  // mean step's at the end; the uniform mode also its step h)
  float aL = 0.0f, aD = 0.0f, aDy = 0.0f, aP = 0.0f, aQ = 0.0f, aR = 0.0f, aG = 0.0f;
  Co cu{};
  float dmu = 0.0f;
  if constexpr (MODE == CK_UNIFORM) {
    cu = md.c0;
    dmu = fmaf(-cu.pj, cu.pk, cu.D);
  }
  for (int blk = nb - 1; blk >= 0; --blk) {
    const int ns = min(CB, n - blk * CB);
    stage_store(a, st, sm.v, sm.h);  // the previous block's readers of v / h finished before its last barrier
    float S2 = ck2, S1j = ck1, S1k = 0.0f;
    lds_sync();
    // recompute the block's states: level 2 before each step in registers, level 1 before each step in LDS
    float S2p[CB];
#pragma unroll
    for (int s = 0; s < CB; ++s) {
      S2p[s] = S2;
      if (s < ns) {
        if (k == 0 && rowl) sm.s1[s][j] = S1j;
        Co c, cd;
        Nd cn;
        if constexpr (MODE == CK_UNIFORM) c = cu;
        else coef_at<MODE>(a, md, lj, lk, sm.h[s], c, cd, cn);
        const float vj = act ? sm.v[s * K + j] : 0.0f;
        const float vk = act ? sm.v[s * K + k] : 0.0f;
        fstep(c, vj, vk, S1j, S1k, S2);
      }
    }
    if (k == 0 && rowl) sm.s1[ns][j] = S1j;
    dma_sync();  // level 1 complete; the block's last cotangent group landed
    // adjoint steps, last first
#pragma unroll
    for (int s = CB - 1; s >= 0; --s) {
      const int g = s / Q;
      if (s % Q == Q - 1) {  // group start: copy the next group's rows (in the last group: the next block's)
        if (g > 0) {
          dma_group(blk, g - 1);
        } else if (blk > 0) {
          dma_group(blk - 1, NG - 1);
          stage_load(a, b, blk - 1, st);
          ck2 = ckp[(size_t)(blk - 1) * (NT + K) + p];
          ck1 = rowl ? ckp[(size_t)(blk - 1) * (NT + K) + NT + j] : 0.0f;
        }
      }
      if (s < ns) {
        const float* grw = sg + (g & 1) * Q * W + (s - g * Q) * W;
        const float G = grw[off_g2] * m_g;  // log rows: -G/2
        const float g2 = LOG ? G * m_u : G;
        const float g1 = grw[off_g1] * m_row;
        float h = 0.0f;
        Co c, cd;
        Nd cn;
        float dm;
        if constexpr (MODE == CK_UNIFORM) {
          c = cu;
          dm = dmu;
        } else {
          h = sm.h[s];
          coef_at<MODE>(a, md, lj, lk, h, c, cd, cn);
          dm = fmaf(-c.pj, c.pk, c.D);
        }
        const float vj = sm.v[s * K + jj] * m_row;
        const float vk = sm.v[s * K + kk] * m_act;
        const float S1pj = sm.s1[s][j];
        const float cj = c.rj * S1pj;
        const float L2 = lam2 + g2;
        const float u = L2 * vk;
        const float t = u * c.pk;
        float xs = t;
        if constexpr (LOG) xs = fmaf(G, sm.s1[s + 1][kk], t);
        const float X = row_sum(xs);
        const float Y = row_sum(u * dm);
        const float gc = lam1 + g1 + X;
        const float colw = add_xor32(L2 * fmaf(c.pk, cj, c.D * vj));
        if ((p & 63) < RS) sm.col[s][w][k] = colw;
        if (k == 0 && rowl) sm.rowp[s][j] = fmaf(c.pj, gc, Y);
        if constexpr (MODE == CK_UNIFORM) {  // sum_t t v_j = phi_k sum_t u v_j with phi_k constant: no aQ
          aL = fmaf(L2, S2p[s], aL);
          aD = fmaf(u, vj, aD);
          aP = fmaf(u, cj, aP);
          aR = fmaf(gc, S1pj, aR);
          aG = fmaf(gc, vj, aG);
        } else if constexpr (MODE == CK_LINEAR) {
          const float hL2 = h * L2, hu = h * u, hgc = h * gc;
          aL = fmaf(hL2, S2p[s], aL);
          aD = fmaf(hu, vj, aD);
          aP = fmaf(hu, cj, aP);
          aQ = fmaf(h * t, vj, aQ);
          aR = fmaf(hgc, S1pj, aR);
          aG = fmaf(hgc, vj, aG);
        } else {
          const float hL2 = h * L2, huv = h * u * vj, hgc = h * gc;
          aL = fmaf(hL2 * S2p[s], cn.L, aL);
          aD = fmaf(huv, cn.Dxy, aD);
          aDy = fmaf(huv, cn.Dy, aDy);
          aP = fmaf(h * u * cj, cn.pk, aP);
          aQ = fmaf(h * t * vj, cn.pj, aQ);
          aR = fmaf(hgc * S1pj, cn.rj, aR);
          aG = fmaf(hgc * vj, cn.pj, aG);
        }
        if constexpr (DH) {
          float dh = L2 * S2p[s] * cd.L;
          dh = fmaf(u * cj, cd.pk, dh);
          dh = fmaf(u * vj, cd.D, dh);
          dh = fmaf(-t * vj, cd.pj, dh);
          dh = fmaf(m_k0 * gc, fmaf(S1pj, cd.rj, vj * cd.pj), dh);
          dh = add_xor32(row_sum(dh));
          if ((p & 63) == 0) sm.dhw[s][w] = dh;
        }
        lam1 = c.rj * gc;
        lam2 = c.L * L2;
      }
      if (s % Q == 0) dma_sync();  // group end: the next group's rows landed (and this group's partials)
    }
    // dv / dh of the block's steps from the staged partials
    for (int e = p; e < ns * K; e += NT) {
      const int ss = e / K, m = e - ss * K;
      float acc = sm.rowp[ss][m];
      for (int ww = 0; ww < nw; ++ww) acc += sm.col[ss][ww][m];
      sm.dv[ss][m] = acc;
    }
    if constexpr (DH) {
      for (int ss = p; ss < ns; ss += NT) {
        float acc = 0.0f;
        for (int ww = 0; ww < nw; ++ww) acc += sm.dhw[ss][ww];
        sm.dh[ss] = acc;
      }
    }
    lds_sync();
    // knots blk*CB + 1 .. blk*CB + ns: dX_t = dv_{t-1} - dv_t (and dtheta_t = dh_{t-1} - dh_t), since
    // v_t = X_{t+1} - X_t; knot 0 gets -dv_0
    const size_t kb = (size_t)b * a.L + (size_t)blk * CB;
    const int nx = (blk + 1) & 1;  // written by the block after this one (zeros for the last)
    for (int e = p; e < ns * K; e += NT) {
      const int s = 1 + e / K, m = e - (s - 1) * K;
      const float hi = s < ns ? sm.dv[s][m] : sm.next[nx][m];
      a.dpath[(kb + s) * a.d + m] = sm.dv[s - 1][m] - hi;
    }
    if constexpr (DH) {
      for (int s = 1 + p; s <= ns; s += NT) a.dclock[kb + s] = sm.dh[s - 1] - (s < ns ? sm.dh[s] : sm.nexth[nx]);
    }
    if (blk == 0) {
      for (int m = p; m < K; m += NT) a.dpath[kb * a.d + m] = -sm.dv[0][m];
      if (DH && p == 0) a.dclock[kb] = -sm.dh[0];
    }
    // for the block before this one (read after its own barriers; the other parity is read above)
    if (p < K) sm.next[blk & 1][p] = sm.dv[0][p];
    if (DH && p == 0) sm.nexth[blk & 1] = sm.dh[0];
  }
  // parameter partials of the sample: dlambda_m = -(sum over the coefficients of channel m of h c'(x) cot(c))
  float grow, gcol;
  float q = row_sum(aQ);  // the phi_j cotangent's per-lane part
  if constexpr (MODE == CK_EXACT) {
    grow = aL + aD;
    gcol = aL + aDy + aP;
    grow = fmaf(m_k0, aR + aG - q, grow);
  } else {  // the node derivatives (and, for the uniform mode, the step) at the mean step
    Co c, cd;
    Nd nd;
    eval_co(a, lj, lk, md.hbar, c, cd, nd);
    const float hs = MODE == CK_UNIFORM ? md.hbar : 1.0f;
    if constexpr (MODE == CK_UNIFORM) q = row_sum(c.pk * aD);
    grow = hs * fmaf(aL, nd.L, aD * nd.Dxy);
    gcol = hs * fmaf(aL, nd.L, fmaf(aD, nd.Dy, aP * nd.pk));
    grow = fmaf(m_k0 * hs, fmaf(aR, nd.rj, (aG - q) * nd.pj), grow);
  }
  const float gr = row_sum(grow);
  if (k == 0 && rowl) sm.grow[j] = gr;
  if (j < MAXK) sm.gcol[j][k] = act ? gcol : 0.0f;
  lds_sync();
  if (p < K) {
    float acc = sm.grow[p];
    for (int qq = 0; qq < K; ++qq) acc += sm.gcol[qq][p];
    a.seqgp[(size_t)b * K + p] = -acc;
  }
}

// One kernel per clock mode (each workgroup returns unless its sample has the kernel's mode): the three bodies
// inlined into one kernel would spill registers. With the clock gradient (DH) every sample takes the exact mode: the
// constant models' step derivatives held in registers would spill beside the block's recomputed states.
template <bool LOG, bool DH, int MODE, int KC>
__global__ __launch_bounds__(1024) void k_seq_bwd(DiagArgs a) {
  static_assert(!DH || MODE == CK_EXACT, "the clock gradient takes exact per-step coefficients");
  __shared__ BwdLds sm;
  extern __shared__ float sg[];
  const int p = threadIdx.x, j = p / RS, k = p % RS;
  const bool act = j < a.K && k < a.K;
  const float lj = act ? a.params[j] : 0.0f, lk = act ? a.params[k] : 0.0f;
  const Clock ck = sample_clock(a, blockIdx.x, sm.red);
  if (!DH && ck.mode != MODE) return;  // uniform across the workgroup: no barrier is left waiting
  Model md{};
  md.hbar = ck.hbar;
  if constexpr (MODE != CK_EXACT) {
    Nd nd;
    eval_co(a, lj, lk, ck.hbar, md.c0, md.c1, nd);
  }
  bwd_body<LOG, DH, MODE, KC>(a, sm, sg, md, lj, lk);
}

// grad_params = the samples' partials summed in a fixed order: one workgroup per channel, its threads striding over
// the samples in float64, then a fixed tree
__global__ __launch_bounds__(256) void k_seq_params(DiagArgs a) {
  __shared__ double red[256];
  const int m = blockIdx.x, t = threadIdx.x;
  double acc = 0.0;
  for (int b = t; b < a.B; b += 256) acc += a.seqgp[(size_t)b * a.K + m];
  red[t] = acc;
  __syncthreads();
  for (int o = 128; o > 0; o >>= 1) {
    if (t < o) red[t] += red[t + o];
    __syncthreads();
  }
  if (t == 0) a.dparams[m] = (float)red[0];
}

}  // namespace seq

int seq_forward(const DiagArgs& a, hipStream_t st) {
  const dim3 grid(a.B), blk(seq_threads(a.K));
  const bool log = a.readout == EWS_READOUT_LOGPREFIX;
  if (a.K == 32) {
    if (log) hipLaunchKernelGGL((seq::k_seq_fwd<true, 32>), grid, blk, 0, st, a);
    else hipLaunchKernelGGL((seq::k_seq_fwd<false, 32>), grid, blk, 0, st, a);
  } else {
    if (log) hipLaunchKernelGGL((seq::k_seq_fwd<true, 0>), grid, blk, 0, st, a);
    else hipLaunchKernelGGL((seq::k_seq_fwd<false, 0>), grid, blk, 0, st, a);
  }
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

template <bool LOG, bool DH, int MODE>
static int launch_bwd(const DiagArgs& a, hipStream_t st) {
  const size_t lds = seq_bwd_lds_bytes(a.W);
  auto kern = a.K == 32 ? seq::k_seq_bwd<LOG, DH, MODE, 32> : seq::k_seq_bwd<LOG, DH, MODE, 0>;
  if (lds > 65536 && hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                         hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) != hipSuccess)
    return -1;
  hipLaunchKernelGGL(kern, dim3(a.B), dim3(seq_threads(a.K)), lds, st, a);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}
template <bool LOG>
static int launch_bwd_all(const DiagArgs& a, hipStream_t st) {
  if (a.dclock) return launch_bwd<LOG, true, seq::CK_EXACT>(a, st);
  if (launch_bwd<LOG, false, seq::CK_UNIFORM>(a, st) != 0) return -1;
  if (launch_bwd<LOG, false, seq::CK_LINEAR>(a, st) != 0) return -1;
  return launch_bwd<LOG, false, seq::CK_EXACT>(a, st);
}

int seq_backward(const DiagArgs& a, hipStream_t st) {
  const int rc = a.readout == EWS_READOUT_LOGPREFIX ? launch_bwd_all<true>(a, st) : launch_bwd_all<false>(a, st);
  if (rc != 0) return -1;
  if (hipGetLastError() != hipSuccess) return -1;
  hipLaunchKernelGGL(seq::k_seq_params, dim3(a.K), dim3(256), 0, st, a);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // namespace ews
