// Pair-group kernels of the rotation-plane EWS scan on MI355X (gfx950): d = 16 (8 planes), depth 2, per-interval
// flows, prefix readout, on chunks whose clock steps are uniform to float32 precision. Every other chunk (and
// every other configuration) runs in the generic kernels of ews_diag.hip.
//
// Math (reference sign, flow exp(-h A)): plane j acts on p_j = v_{2j} + i v_{2j+1}; with x_j = h u_j,
// u_j = -conj(z_j), rho_j = e^{x_j}, phi_j = exp[0, x_j]:
//     S1_j  <- rho_j S1_j + phi_j p_j
//     SB_jk <- LB_jk SB_jk + c_j phi_k p_k       + IB_jk p_j p_k          LB = e^{h (u_j + u_k)}
//     SA_jk <- LA_jk SA_jk + c_j conj(phi_k p_k) + IA_jk p_j conj(p_k)    LA = e^{h (u_j + conj(u_k))}
// with c_j = rho_j S1_j (before the update), IB = exp[0, x_j, h (u_j + u_k)], IA = exp[0, x_j, h (u_j + conj u_k)]:
// the Chen step S2 <- M S2 M^T + (M S1) s1^T + s2 (ews/core/chen_scan.py:124-152) diagonalised plane by plane,
// with the closed-form local terms of ews/core/kernels/plane_engine.py:134-152.
//
// Lane layout. A chunk of T intervals belongs to a group of G = 8 * (8 / KP) lanes: lane (j, kg) = 8 kg + j owns
// plane j's level 1 and the KP level-2 pairs (j, k), k = KP kg .. KP kg + KP - 1. A wavefront (= one workgroup) holds
// 64 / G groups: consecutive chunks of one sample. The forward and the local adjoint use KP = 4 (16-lane groups);
// the full adjoint, which carries four times the live values per pair, uses KP = 2 (32-lane groups). The row sums
// over k that feed the level-1 adjoint are DPP / swizzle adds among the lanes of plane j; the column sums over j
// (gradients of the later factor) go through LDS once per block of steps, off the sequential chain.
//
// Uniform chunks. When every step h_t of a chunk, and every partial sum of (h_t - hbar), is within
// 2^-21 / max|u| of the chunk mean hbar (as with a float32 uniform clock), every coefficient is taken at hbar:
// relative error <= 2^-21 per coefficient and <= 2^-20 on a product of flows, since the partial sums of the steps
// telescope to clock differences. Parameter gradients, whose h-factor enters linearly, weight each step by its own
// h_t.
//
// Scaling. Level-2 pair states are kept halved (SAh = SA/2, SBh = SB/2), so an output block is sums and
// differences of them, and level-2 cotangents doubled (lA = 2 dL/dSA, lB = 2 dL/dSB); the halves fold into the
// coefficients (phih = phi/2, IBh = IB/2, ...).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <type_traits>

#include "ews_args.h"
#include "ews_hip.h"
#include "ews_lanes.h"
#include "ews_numerics.h"
#include "ews_pairs.h"

namespace ews {
namespace pairs {

constexpr int K = 8;      // planes
constexpr int DIM = 16;   // channels
constexpr int NB = 4;     // steps per block of the full adjoint's column sums
// look-back forward (k_fwd_lb)
constexpr int kSpinLimit = 1 << 20;  // polls of a status word before the look-back gives up (rows turn NaN)
constexpr int LBB = 4;               // aggregates whose loads are in flight together in the look-back
constexpr int LBG = 8;               // quads per look-back group
// a bit pattern no arithmetic here produces (a signalling NaN with a payload): a look-back aggregate word not yet
// published
constexpr unsigned long long kLbEmpty = 0x7FF4E3A5C0DE0000ull;
constexpr int LBT = 32;              // words between the samples' ticket counters (one per 128-byte line)
constexpr int VPITCH = (kMaxT + 1) * DIM;  // LDS floats per group of staged increments (one padding row)

template <int KP> struct Geo {
  static constexpr int NKG = K / KP;  // k-groups per plane row
  static constexpr int G = K * NKG;   // lanes per chunk group
  static constexpr int GPW = 64 / G;  // chunk groups per wavefront (workgroup)
};

typedef float f4u __attribute__((ext_vector_type(4), aligned(4)));
typedef float f2u __attribute__((ext_vector_type(2), aligned(4)));
typedef float f4a __attribute__((ext_vector_type(4)));

__device__ __forceinline__ cf cjm(cf a, cf b) { return cf{a.re * b.re + a.im * b.im, a.re * b.im - a.im * b.re}; }  // conj(a) b
__device__ __forceinline__ float redot(cf a, cf b) { return a.re * b.re + a.im * b.im; }  // Re(conj(a) b)
__device__ __forceinline__ cf fma_c(cf a, cf b, cf c) {  // a b + c
  return cf{fmaf(a.re, b.re, fmaf(-a.im, b.im, c.re)), fmaf(a.re, b.im, fmaf(a.im, b.re, c.im))};
}

// cross-lane moves: DPP row_ror inside rows of 16 lanes (bound_ctrl with a zero old value, so that the move folds
// into the consuming add as its DPP source), v_permlane16_swap for lane ^ 16 (a VALU op: no LDS round trip)
#define EWS_ROR(v, n) __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x120 + (n), 0xf, 0xf, true))
// v[lane] + v[lane ^ 16] in every lane: the swap exchanges the odd rows of one copy with the even rows of the other
__device__ __forceinline__ float add_xor16(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// sum over the k-groups of plane j (lanes j + 8 kg of the group)
template <int KP> __device__ __forceinline__ float kg_sum(float v) {
  if constexpr (Geo<KP>::NKG >= 2) v += EWS_ROR(v, 8);
  if constexpr (Geo<KP>::NKG >= 4) v = add_xor16(v);
  return v;
}
template <int KP> __device__ __forceinline__ cf kg_sum(cf v) { return cf{kg_sum<KP>(v.re), kg_sum<KP>(v.im)}; }

// Compile-time loop: the pair arrays below stay in registers only if every index is a constant.
template <int I, int N, class F> __device__ __forceinline__ void static_for(F&& f) {
  if constexpr (I < N) {
    f(std::integral_constant<int, I>{});
    static_for<I + 1, N>(f);
  }
}

// Compile-time loop I, I-1, ..., 0.
template <int I, class F> __device__ __forceinline__ void static_down(F&& f) {
  if constexpr (I >= 0) {
    f(std::integral_constant<int, I>{});
    static_down<I - 1>(f);
  }
}

struct Lane {
  int gi, gl, j, kg;
};
template <int KP> __device__ __forceinline__ Lane lane_of(int tid) {
  Lane l;
  l.gi = tid / Geo<KP>::G;
  l.gl = tid % Geo<KP>::G;
  l.j = l.gl & 7;
  l.kg = l.gl >> 3;
  return l;
}

__device__ __forceinline__ cf load_u(const float* params, int j) { return cf{-params[2 * j], params[2 * j + 1]}; }

// Increments v_i = X_{i+1} - X_i of the workgroup's intervals into LDS, group gi's interval t at
// s_v[gi * VPITCH + 16 t]; clock steps into s_h[gi * kMaxT + t] when s_h is given.
template <int KP, bool BF16>
__device__ __forceinline__ void stage(const DiagArgs& a, int b, int cb, float* s_v, float* s_h) {
  constexpr int GPW = Geo<KP>::GPW, U = 8;  // U loads per operand in flight per thread before any LDS write
  const int i0 = cb * a.T;
  const int n = min(GPW * a.T, a.n_int - i0);
  const int tid = threadIdx.x;
  if constexpr (!BF16) {
    const float* src = reinterpret_cast<const float*>(a.path) + ((size_t)b * a.L + i0) * DIM;
    for (int qb = tid; qb < n * 4; qb += U * 64) {
      f4a x0[U], x1[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int q = qb + u * 64, i = q >> 2, c4 = q & 3;
        if (q < n * 4) {
          x0[u] = *reinterpret_cast<const f4a*>(src + (size_t)i * DIM + 4 * c4);
          x1[u] = *reinterpret_cast<const f4a*>(src + (size_t)(i + 1) * DIM + 4 * c4);
        }
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int q = qb + u * 64, i = q >> 2, c4 = q & 3;
        if (q < n * 4) {
          const int gi = i / a.T, t = i - gi * a.T;
          *reinterpret_cast<f4a*>(s_v + gi * VPITCH + t * DIM + 4 * c4) = x1[u] - x0[u];
        }
      }
    }
  } else {
    const unsigned short* src = reinterpret_cast<const unsigned short*>(a.path) + ((size_t)b * a.L + i0) * DIM;
    for (int qb = tid; qb < n * DIM; qb += U * 64) {
      unsigned short x0[U], x1[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int q = qb + u * 64, i = q / DIM, ch = q - i * DIM;
        if (q < n * DIM) {
          x0[u] = src[(size_t)i * DIM + ch];
          x1[u] = src[(size_t)(i + 1) * DIM + ch];
        }
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int q = qb + u * 64, i = q / DIM, ch = q - i * DIM;
        if (q < n * DIM) {
          const int gi = i / a.T, t = i - gi * a.T;
          s_v[gi * VPITCH + t * DIM + ch] =
              __uint_as_float(((unsigned)x1[u]) << 16) - __uint_as_float(((unsigned)x0[u]) << 16);
        }
      }
    }
  }
  if (s_h) {
    const float* th = a.clock + (size_t)b * a.L + i0;
    for (int ib = tid; ib < n; ib += 4 * 64) {
      float y0[4], y1[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int i = ib + u * 64;
        if (i < n) {
          y0[u] = th[i];
          y1[u] = th[i + 1];
        }
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int i = ib + u * 64;
        if (i < n) {
          const int gi = i / a.T, t = i - gi * a.T;
          s_h[gi * kMaxT + t] = y1[u] - y0[u];
        }
      }
    }
  }
}

// Block staging of increments: SB steps of every group of the workgroup at a time, double-buffered in LDS
// (buffer (blk & 1), group gi's step s at gi * VBLK + s * DIM). The loads of the next block are issued into
// registers before the current block's steps and written to LDS after them, so the staging latency hides
// behind SB steps and the LDS footprint stays at 2 x GPW x SB x 64 bytes.
constexpr int SB = 16;           // steps per staged block
constexpr int VBLK = SB * DIM;   // LDS floats per group and block buffer
template <int GPW, bool BF16> struct VRaw {
  static constexpr int IPS = BF16 ? 2 : 4;                  // 16-byte items per step
  static constexpr int NI = (GPW * SB * IPS + 63) / 64;     // items per lane
  f4a x0[NI], x1[NI];                                       // knots x_i, x_{i+1} (bf16: raw bits)
};
template <int GPW, bool BF16>
__device__ __forceinline__ bool vblk_item(const DiagArgs& a, int cb, int blk, int item, int& gi, int& st, int& q,
                                          int& idx) {
  constexpr int IPS = VRaw<GPW, BF16>::IPS;
  gi = item / (SB * IPS);
  const int rem = item - gi * (SB * IPS);
  st = rem / IPS;
  q = rem - st * IPS;
  const int c = cb + gi, t = blk * SB + st;
  idx = c * a.T + t;
  return item < GPW * SB * IPS && c < a.C && t < a.T && idx < a.n_int;
}
template <int GPW, bool BF16>
__device__ __forceinline__ void vblk_load(const DiagArgs& a, int b, int cb, int blk, VRaw<GPW, BF16>& r) {
#pragma unroll
  for (int i = 0; i < VRaw<GPW, BF16>::NI; ++i) {
    int gi, st, q, idx;
    if (vblk_item<GPW, BF16>(a, cb, blk, (int)threadIdx.x + 64 * i, gi, st, q, idx)) {
      const char* row = reinterpret_cast<const char*>(a.path) + ((size_t)b * a.L + idx) * DIM * (BF16 ? 2 : 4);
      r.x0[i] = *reinterpret_cast<const f4a*>(row + 16 * q);
      r.x1[i] = *reinterpret_cast<const f4a*>(row + DIM * (BF16 ? 2 : 4) + 16 * q);
    }
  }
}
__device__ __forceinline__ float bf_lo(float w) { return __uint_as_float(__float_as_uint(w) << 16); }
__device__ __forceinline__ float bf_hi(float w) { return __uint_as_float(__float_as_uint(w) & 0xffff0000u); }
template <int GPW, bool BF16>
__device__ __forceinline__ void vblk_store(const DiagArgs& a, int cb, int blk, const VRaw<GPW, BF16>& r,
                                           float* buf) {
#pragma unroll
  for (int i = 0; i < VRaw<GPW, BF16>::NI; ++i) {
    int gi, st, q, idx;
    if (vblk_item<GPW, BF16>(a, cb, blk, (int)threadIdx.x + 64 * i, gi, st, q, idx)) {
      float* o = buf + gi * VBLK + st * DIM;
      if constexpr (!BF16) {
        *reinterpret_cast<f4a*>(o + 4 * q) = r.x1[i] - r.x0[i];
      } else {  // 8 bf16 channels 8q .. 8q + 7, little-endian pairs
        const f4a u = r.x0[i], w = r.x1[i];
        *reinterpret_cast<f4a*>(o + 8 * q) =
            f4a{bf_lo(w.x) - bf_lo(u.x), bf_hi(w.x) - bf_hi(u.x), bf_lo(w.y) - bf_lo(u.y), bf_hi(w.y) - bf_hi(u.y)};
        *reinterpret_cast<f4a*>(o + 8 * q + 4) =
            f4a{bf_lo(w.z) - bf_lo(u.z), bf_hi(w.z) - bf_hi(u.z), bf_lo(w.w) - bf_lo(u.w), bf_hi(w.w) - bf_hi(u.w)};
      }
    }
  }
}

// p_j and the lane's KP p_k of step t
template <int KP> __device__ __forceinline__ void load_p(const float* vr, const Lane& l, cf& pj, cf* pk) {
  const float2 a = *reinterpret_cast<const float2*>(vr + 2 * l.j);
  pj = cf{a.x, a.y};
  static_for<0, KP / 2>([&](auto ic) {
    constexpr int i = ic;
    const f4a v = *reinterpret_cast<const f4a*>(vr + 2 * KP * l.kg + 4 * i);
    pk[2 * i] = cf{v.x, v.y};
    pk[2 * i + 1] = cf{v.z, v.w};
  });
}

// Level-2 part of a readout row (d^2 = 256 floats from off2) moved between HBM and the lane slices through a
// per-group LDS buffer of 256 floats, so that every global access instruction of a group covers a contiguous run
// (G lanes x 16 bytes) instead of scattered 16-byte pieces: lane gl moves pieces gl, gl + G, ... of the row.
// The buffer holds the 16 x 16 block row-major with 4 floats of padding after every pair of rows (row r at
// 16 r + 4 (r >> 1)): the lanes (j = 0..7) of one LDS cycle then start their row 2j slices on distinct bank
// quads (the unpadded pitch puts all eight on one quad), and the contiguous pieces stay conflict-free too.
// The lane slice of (j, kg) is row 2j (buffer [36 j, 36 j + 16)) and row 2j + 1 ([36 j + 16, 36 j + 32)),
// columns 2 KP kg .. 2 KP kg + 2 KP - 1. LDS operations of one wavefront execute in program order, so a
// compiler barrier between the write and the read of another lane's data is enough.
constexpr int RBUF = DIM * DIM + 2 * DIM;  // floats of the padded 16 x 16 block
__device__ __forceinline__ int piece_at(int pi) { return 4 * pi + 4 * (pi >> 3); }  // piece pi = row pi/4, col 4(pi%4)
__device__ __forceinline__ int row_at(int r) { return DIM * r + 4 * (r >> 1); }
template <int KP> struct Pieces {
  static constexpr int NP = 64 / Geo<KP>::G;  // 16-byte pieces per lane
  f4u v[NP];
};
template <int KP> __device__ __forceinline__ Pieces<KP> load_pieces(const float* row2, int gl) {
  Pieces<KP> pc;
  static_for<0, Pieces<KP>::NP>([&](auto ic) {
    constexpr int i = ic;
    pc.v[i] = *reinterpret_cast<const f4u*>(row2 + 4 * (gl + Geo<KP>::G * i));
  });
  return pc;
}
template <int KP> __device__ __forceinline__ void pieces_to_lds(const Pieces<KP>& pc, float* buf, int gl) {
  static_for<0, Pieces<KP>::NP>([&](auto ic) {
    constexpr int i = ic;
    *reinterpret_cast<f4a*>(buf + piece_at(gl + Geo<KP>::G * i)) = f4a{pc.v[i].x, pc.v[i].y, pc.v[i].z, pc.v[i].w};
  });
}
__device__ __forceinline__ void wave_order() { __builtin_amdgcn_wave_barrier(); }

// products p_j p_k and p_j conj(p_k)
__device__ __forceinline__ void prods(cf pj, cf pk, cf& pi, cf& pic) {
  const float aa = pj.re * pk.re, bb = pj.im * pk.im, cc = pj.re * pk.im, dd = pj.im * pk.re;
  pi = cf{aa - bb, cc + dd};
  pic = cf{aa + bb, dd - cc};
}

// ------------------------------------------------------------------------------------------------ coefficient table
// Every coefficient at one reference step h0 (the mean step of chunk 0 of sample 0): chunks whose mean step hbar
// is within 2^-22 / max|u| of h0 (every chunk of a uniform clock) take the table instead of evaluating the
// divided differences themselves. Flows are corrected to first order, c(hbar) = c(h0) + c'(h0) (hbar - h0)
// (their errors compound over the chunk's steps; the second-order remainder is below 2^-44); every other
// coefficient is used at h0 (relative error <= 2^-22).
// Layout (complex floats after a 16-float header holding h0): per plane p, entry e at 16 + 2 (9 p + e);
// per pair 8 j + k, entry e at 16 + 2 * 72 + 2 (16 (8 j + k) + e).
enum { TP_RHO, TP_RHO1, TP_RHOI, TP_RHOI1, TP_PHI, TP_PHI1, TP_DPHI, TP_PHIH, TP_PHI1H };
enum { TQ_LB, TQ_LB1, TQ_LA, TQ_LA1, TQ_LBI, TQ_LBI1, TQ_LAI, TQ_LAI1, TQ_IB, TQ_IA, TQ_IB1, TQ_IA1, TQ_DXB, TQ_DYB,
       TQ_DXA, TQ_DYA };
__device__ __forceinline__ cf tp(const float* tab, int p, int e) {
  const float2 v = *reinterpret_cast<const float2*>(tab + 16 + 2 * (9 * p + e));
  return cf{v.x, v.y};
}
__device__ __forceinline__ cf tq(const float* tab, int j, int k, int e) {
  const float2 v = *reinterpret_cast<const float2*>(tab + 16 + 2 * 72 + 2 * (16 * (8 * j + k) + e));
  return cf{v.x, v.y};
}
__device__ __forceinline__ void stp(float* tab, int p, int e, cf v) {
  *reinterpret_cast<float2*>(tab + 16 + 2 * (9 * p + e)) = float2{v.re, v.im};
}
__device__ __forceinline__ void stq(float* tab, int j, int k, int e, cf v) {
  *reinterpret_cast<float2*>(tab + 16 + 2 * 72 + 2 * (16 * (8 * j + k) + e)) = float2{v.re, v.im};
}
// reference step: the mean step of chunk 0 of sample 0, in the classification's arithmetic
__device__ __forceinline__ float ref_step(const DiagArgs& a) {
  const int Tc = min(a.T, a.n_int);
  return (a.clock[Tc] - a.clock[0]) / (float)Tc;
}
// Three wavefronts share the entries (a single chain of series and exponentials per lane otherwise): wavefront 0
// the plane nodes and the pair flows, 1 the B-pair divided differences, 2 the A-pair ones.
__global__ __launch_bounds__(192) void k_coef_table(DiagArgs a) {
  if (blockIdx.x > 0) {  // the other workgroups fill the look-back aggregates with the "not yet published" sentinel
    const size_t n = (size_t)a.B * (a.NQ + (a.NQ + LBG - 1) / LBG) * (a.D + 2 * K);
    unsigned long long* w = reinterpret_cast<unsigned long long*>(a.lbagg);
    for (size_t i = (size_t)(blockIdx.x - 1) * blockDim.x + threadIdx.x; i < n; i += (size_t)(gridDim.x - 1) * blockDim.x)
      w[i] = kLbEmpty;
    return;
  }
  // the look-back forward's status words (quads, then groups of LBG quads) and its ticket start at zero (this
  // launch runs first)
  const int nwords = a.B * (a.NQ + (a.NQ + LBG - 1) / LBG) + a.B * LBT;
  for (int i = threadIdx.x; i < nwords; i += blockDim.x) a.lbflag[i] = 0;
  const int role = threadIdx.x >> 6, l = threadIdx.x & 63;
  const int j = l >> 3, k = l & 7;
  float* tab = a.ctab;
  const float h0 = ref_step(a);
  const cf uj = load_u(a.params, j), uk = load_u(a.params, k);
  const cf xj = h0 * uj;
  const cf ub = uj + uk, ua = uj + conj(uk);
  if (role == 0) {
    if (l == 0) {  // header: the reference step, max |u_j| and max d_j (the chunk classification's bounds)
      float R = 0.0f, Dm = 0.0f;
      for (int p = 0; p < K; ++p) {
        R = fmaxf(R, absv(load_u(a.params, p)));
        Dm = fmaxf(Dm, a.params[2 * p]);
      }
      tab[0] = h0;
      tab[1] = R;
      tab[2] = Dm;
      reinterpret_cast<int*>(tab)[kCtabStatus] = 0;  // the look-back forward's error word
    }
    if (k == 0) {
      const Node1<cf> nj = node1(xj);
      const cf ri = expv(-xj);
      stp(tab, j, TP_RHO, nj.e);
      stp(tab, j, TP_RHO1, nj.e * uj);
      stp(tab, j, TP_RHOI, ri);
      stp(tab, j, TP_RHOI1, -(ri * uj));
      stp(tab, j, TP_PHI, nj.p);
      stp(tab, j, TP_PHI1, nj.dp * uj);
      stp(tab, j, TP_DPHI, nj.dp);
      stp(tab, j, TP_PHIH, 0.5f * nj.p);
      stp(tab, j, TP_PHI1H, 0.5f * (nj.dp * uj));
    }
    const cf LB = expv(h0 * ub), LA = expv(h0 * ua), LBi = expv(-(h0 * ub)), LAi = expv(-(h0 * ua));
    stq(tab, j, k, TQ_LB, LB);
    stq(tab, j, k, TQ_LB1, LB * ub);
    stq(tab, j, k, TQ_LA, LA);
    stq(tab, j, k, TQ_LA1, LA * ua);
    stq(tab, j, k, TQ_LBI, LBi);
    stq(tab, j, k, TQ_LBI1, -(LBi * ub));
    stq(tab, j, k, TQ_LAI, LAi);
    stq(tab, j, k, TQ_LAI1, -(LAi * ua));
  } else if (role == 1) {
    const DD3<cf> db = dd3<cf, true>(xj, h0 * ub);
    stq(tab, j, k, TQ_IB, 0.5f * db.d);
    stq(tab, j, k, TQ_IB1, 0.5f * (db.dx * uj + db.dy * ub));
    stq(tab, j, k, TQ_DXB, db.dx);
    stq(tab, j, k, TQ_DYB, db.dy);
  } else {
    const DD3<cf> da = dd3<cf, true>(xj, h0 * ua);
    stq(tab, j, k, TQ_IA, 0.5f * da.d);
    stq(tab, j, k, TQ_IA1, 0.5f * (da.dx * uj + da.dy * ua));
    stq(tab, j, k, TQ_DXA, da.dx);
    stq(tab, j, k, TQ_DYA, da.dy);
  }
}
// first-order flow from the table: c(h0) + c'(h0) dlt
__device__ __forceinline__ cf tflow(cf c0, cf c1, float dlt) { return cf{fmaf(c1.re, dlt, c0.re), fmaf(c1.im, dlt, c0.im)}; }

// Forward coefficients of the lane at the chunk's mean step.
template <int KP> struct FwdCoef {
  cf rho, phi;            // plane j
  cf phk[KP];             // phi_k / 2
  cf LB[KP], LA[KP];      // pair flows
  cf IB[KP], IA[KP];      // IB / 2, IA / 2
};
template <int KP>
__device__ __forceinline__ void fwd_coef(const DiagArgs& a, const Lane& l, float hb, bool use_tab, FwdCoef<KP>& f) {
  if (use_tab) {
    const float* tab = a.ctab;
    const float dlt = hb - tab[0];
    f.rho = tflow(tp(tab, l.j, TP_RHO), tp(tab, l.j, TP_RHO1), dlt);
    f.phi = tp(tab, l.j, TP_PHI);
    static_for<0, KP>([&](auto qc) {
      constexpr int q = qc;
      const int k = KP * l.kg + q;
      f.phk[q] = tp(tab, k, TP_PHIH);
      f.LB[q] = tflow(tq(tab, l.j, k, TQ_LB), tq(tab, l.j, k, TQ_LB1), dlt);
      f.LA[q] = tflow(tq(tab, l.j, k, TQ_LA), tq(tab, l.j, k, TQ_LA1), dlt);
      f.IB[q] = tq(tab, l.j, k, TQ_IB);
      f.IA[q] = tq(tab, l.j, k, TQ_IA);
    });
    return;
  }
  const cf uj = load_u(a.params, l.j);
  const cf xj = hb * uj;
  const Node1<cf> nj = node1(xj);
  f.rho = nj.e;
  f.phi = nj.p;
  static_for<0, KP>([&](auto qc) {
    constexpr int q = qc;
    const cf uk = load_u(a.params, KP * l.kg + q);
    const Node1<cf> nk = node1(hb * uk);
    f.phk[q] = 0.5f * nk.p;
    const cf ub = uj + uk, ua = uj + conj(uk);
    f.LB[q] = expv(hb * ub);
    f.LA[q] = expv(hb * ua);
    f.IB[q] = 0.5f * dd3<cf, false>(xj, hb * ub).d;
    f.IA[q] = 0.5f * dd3<cf, false>(xj, hb * ua).d;
  });
}

// ------------------------------------------------------------------------------------------------ classification
// Chunk c of sample b: flag bit 0 = uniform steps (coefficients at the mean step hbar), bit 1 = the steps may be
// inverted backwards (stepping back amplifies errors by e^{2 Dmax tau} <= 2 over the chunk). Evaluated by the 16
// lanes of the chunk's group, each over every 16th step, then combined with DPP inside the group.
__device__ __forceinline__ float row_max16(float v) {
  v = fmaxf(v, EWS_ROR(v, 8));
  v = fmaxf(v, EWS_ROR(v, 4));
  v = fmaxf(v, EWS_ROR(v, 2));
  v = fmaxf(v, EWS_ROR(v, 1));
  return v;
}
__device__ __forceinline__ int classify_chunk(const DiagArgs& a, int b, int c, int gl, float& hb) {
  constexpr int U = kMaxT / 16;
  const int t0 = c * a.T, Tc = min(a.T, a.n_int - t0);
  const float* th = a.clock + (size_t)b * a.L + t0;
  const float R = a.ctab[1], Dm = a.ctab[2];  // max |u_j| and max d_j, from the coefficient table's header
  float x0[U], x1[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {  // every clock load in flight before the first use
    const int t = gl + 16 * u;
    x0[u] = t < Tc ? th[t] : 0.0f;
    x1[u] = t < Tc ? th[t + 1] : 0.0f;
  }
  const float th0 = th[0];
  const float tau = th[Tc] - th0;
  hb = tau / (float)Tc;
  float dev = 0.0f, drift = 0.0f, bad = 0.0f;
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int t = gl + 16 * u;
    if (t < Tc) {
      const float h = x1[u] - x0[u];
      if (!isfinite(h)) bad = 1.0f;
      dev = fmaxf(dev, fabsf(h - hb));
      drift = fmaxf(drift, fabsf((x1[u] - th0) - (float)(t + 1) * hb));
    }
  }
  dev = row_max16(dev);
  drift = row_max16(drift);
  bad = row_max16(bad);
  const bool fin = bad == 0.0f && isfinite(tau) && isfinite(R);
  const float lim = 4.76837158e-7f;  // 2^-21
  const bool uni = fin && R * dev <= lim && R * drift <= lim;
  const bool inv = fin && 2.0f * Dm * fabsf(tau) <= 0.69314718f;
  const bool tab = uni && R * fabsf(hb - a.ctab[0]) <= 0.5f * lim;  // the coefficient table applies
  return (uni ? 1 : 0) | (inv ? 2 : 0) | (tab ? 4 : 0);
}

// ------------------------------------------------------------------------------------------------ carries
// Float64 Chen combine of the chunk summaries in quads of four chunks (the chunks of one forward workgroup):
// every quad's summary in parallel (k_quad_fwd_agg), one blocked scan over the quads of each sample
// (k_quad_fwd_scan), and the carries inside a quad rebuilt by the prefix-row kernel from the quad's carry
// (at most three combines). The adjoint carries mirror it (k_quad_bwd_agg / k_quad_bwd_scan / full adjoint).
// Lane view of these kernels: 64 lanes, lane = 8 j + k holds level 1 of plane j and the pair (j, k).
struct dc {
  double re, im;
};
__device__ __forceinline__ dc operator+(dc a, dc b) { return dc{a.re + b.re, a.im + b.im}; }
__device__ __forceinline__ dc operator-(dc a, dc b) { return dc{a.re - b.re, a.im - b.im}; }
__device__ __forceinline__ dc operator*(dc a, dc b) { return dc{a.re * b.re - a.im * b.im, a.re * b.im + a.im * b.re}; }
__device__ __forceinline__ dc cjd(dc a) { return dc{a.re, -a.im}; }
__device__ __forceinline__ dc dexpc(dc x) {
  double sn, cs;
  sincos(x.im, &sn, &cs);
  const double m = exp(x.re);
  return dc{m * cs, m * sn};
}
__device__ __forceinline__ dc ld_fd(const float* p) { return dc{(double)p[0], (double)p[1]}; }
__device__ __forceinline__ dc ld_dd(const double* p) { return dc{p[0], p[1]}; }
__device__ __forceinline__ void st_dd(double* p, dc v) {
  p[0] = v.re;
  p[1] = v.im;
}
__device__ __forceinline__ void st_fd(float* p, dc v) {
  p[0] = (float)v.re;
  p[1] = (float)v.im;
}
__device__ __forceinline__ dc rowsum8(dc v) {  // over lanes 8 j .. 8 j + 7 (DPP)
  return dc{lanes::sum8(v.re), lanes::sum8(v.im)};
}
// flow exp(u_p tau) of plane p over the clock span of chunks [c0, c1) (per-interval flows)
__device__ __forceinline__ dc span_flow(const DiagArgs& a, int b, int c0, int c1, int p) {
  const float* th = a.clock + (size_t)b * a.L;
  const double tau = (double)th[min(c1 * a.T, a.n_int)] - (double)th[c0 * a.T];
  return dexpc(dc{-(double)a.params[2 * p] * tau, (double)a.params[2 * p + 1] * tau});
}

struct PairSt {
  dc S1, SA, SB;
};
__device__ __forceinline__ int poff(int j, int k) { return DIM + 4 * (8 * j + k); }
__device__ __forceinline__ PairSt load_st_d(const double* row, int j, int k) {
  return PairSt{ld_dd(row + 2 * j), ld_dd(row + poff(j, k)), ld_dd(row + poff(j, k) + 2)};
}
__device__ __forceinline__ PairSt load_st_f(const float* row, int j, int k) {
  return PairSt{ld_fd(row + 2 * j), ld_fd(row + poff(j, k)), ld_fd(row + poff(j, k) + 2)};
}
__device__ __forceinline__ void store_st_d(double* row, int j, int k, const PairSt& s) {
  if (k == 0) st_dd(row + 2 * j, s.S1);
  st_dd(row + poff(j, k), s.SA);
  st_dd(row + poff(j, k) + 2, s.SB);
}
__device__ __forceinline__ void store_st_f(float* row, int j, int k, const PairSt& s) {
  if (k == 0) st_fd(row + 2 * j, s.S1);
  st_fd(row + poff(j, k), s.SA);
  st_fd(row + poff(j, k) + 2, s.SB);
}
// S <- (flow F applied to S) (x) Y: the Chen product with a summary Y (level 1 y1j, y1k; pair yA, yB)
__device__ __forceinline__ void chen_d(PairSt& s, dc Fj, dc Fk, dc y1j, dc y1k, dc yA, dc yB) {
  const dc cj = Fj * s.S1;
  s.SA = (Fj * cjd(Fk)) * s.SA + cj * cjd(y1k) + yA;
  s.SB = (Fj * Fk) * s.SB + cj * y1k + yB;
  s.S1 = cj + y1j;
}
// X <- J^T X for the transfer of a summary with flow F and level-1 increment l1 (then add the local part)
__device__ __forceinline__ void adj_d(PairSt& X, dc Fj, dc Fk, dc l1k) {
  const dc toC = rowsum8(cjd(l1k) * X.SB + l1k * X.SA);
  X.SB = cjd(Fj * Fk) * X.SB;
  X.SA = cjd(Fj * cjd(Fk)) * X.SA;
  X.S1 = cjd(Fj) * (X.S1 + toC);
}
__device__ __forceinline__ void add_st(PairSt& X, const PairSt& m) {
  X.S1 = X.S1 + m.S1;
  X.SA = X.SA + m.SA;
  X.SB = X.SB + m.SB;
}
// <m, D s> of a cotangent m and a state s (pair layout), D the derivation d/dh of the flows (level 1 of plane j
// times u_j, pair (j, k) SB times u_j + u_k and SA times u_j + conj(u_k)): the lane's share, float64 (lanes
// k = 0 add the level-1 term)
__device__ __forceinline__ double flow_dot(const DiagArgs& a, const PairSt& m, const PairSt& s, int j, int k) {
  const dc uj{-(double)a.params[2 * j], (double)a.params[2 * j + 1]};
  const dc uk{-(double)a.params[2 * k], (double)a.params[2 * k + 1]};
  const dc tB = cjd(m.SB) * ((uj + uk) * s.SB), tA = cjd(m.SA) * ((uj + cjd(uk)) * s.SA);
  double r = tB.re + tA.re;
  if (k == 0) r += (cjd(m.S1) * (uj * s.S1)).re;
  return r;
}
__device__ __forceinline__ double wave_sum_d(double v) { return lanes::sum64(v); }

// level-1 increment of the span [ca, cb) of plane p: carry1(cb) - F carry1(ca)
__device__ __forceinline__ dc l1_inc(const DiagArgs& a, int b, int ca, int cb, int p, dc F) {
  const double* c0 = a.carries + ((size_t)b * (a.C + 1) + ca) * a.D;
  const double* c1 = a.carries + ((size_t)b * (a.C + 1) + cb) * a.D;
  return ld_dd(c1 + 2 * p) - F * ld_dd(c0 + 2 * p);
}

// chunk flows of the quad (LDS + cflow) and the quad flow (qflow)
__device__ __forceinline__ void quad_flows(const DiagArgs& a, int b, int q, int c0, int nc, dc (*s_F)[K]) {
  const int l = threadIdx.x;
  if (l < 8 * nc) {
    const int i = l >> 3, p = l & 7;
    const dc F = span_flow(a, b, c0 + i, c0 + i + 1, p);
    s_F[i][p] = F;
    st_dd(a.cflow + (((size_t)b * a.C + c0 + i) * K + p) * 2, F);
  } else if (l >= 32 && l < 32 + K) {
    const int p = l - 32;
    st_dd(a.qflow + (((size_t)b * a.NQ + q) * K + p) * 2, span_flow(a, b, c0, c0 + nc, p));
  }
  __syncthreads();
}

// Scans over the quads of one sample, one workgroup of SW wavefronts per sample. The quad inputs are staged into
// LDS a segment of up to SSEG quads at a time by the whole workgroup; the segment's quads are split into SW blocks
// of consecutive quads, one per wavefront:
//   1. every wavefront combines its block from a zero state (the block's summary and flow);
//   2. wavefront 0 chains the SW block summaries from the segment's carry (the block carries);
//   3. every wavefront rescans its block from its block carry and writes the carry of each quad.
// The float64 dependency chain per segment is thus (block length) + SW + (block length) combines instead of one
// per quad (26 instead of 71 at c2). Every wavefront reads its next operands from LDS while the current combine
// runs. Lane view: lane = 8 j + k holds level 1 of plane j and the pair (j, k).
constexpr int SW = 8;                       // wavefronts of a scan workgroup
constexpr int SBQ = 9;                      // quads per wavefront block of a full segment
constexpr int SSEG = SW * SBQ;              // quads per staged segment
constexpr int QROW = DIM + DIM * DIM;       // floats of a quad's state
struct ScanLds {
  float y[SSEG][QROW];                      // quad summary / adjoint aggregate (float32)
  dc F[SSEG][K];                            // quad flows
  dc l1[SSEG][K];                           // quad level-1 increments (adjoint scan)
  dc bS1[SW][64], bSA[SW][64], bSB[SW][64]; // per block: summary (phase 1), then carry (phase 2), lane layout
  dc bF[SW][K];                             // block flows
  dc bl1[SW][K];                            // block level-1 increments (adjoint scan)
};
constexpr size_t kScanLds = sizeof(ScanLds);
// Every load of the segment is in flight at once (the flows and level-1 increments first, then all of the rows:
// at most SSEG * QROW / 4 float4 over SW * 64 threads), and only then written to LDS.
__device__ __forceinline__ void stage_seg(const DiagArgs& a, int b, int q0, int nq, bool with_l1, ScanLds& sg) {
  constexpr int NT = SW * 64, R4 = QROW / 4, U = (SSEG * R4 + NT - 1) / NT, UF = (SSEG * K + NT - 1) / NT;
  const double* fs = a.qflow + ((size_t)b * a.NQ + q0) * K * 2;
  const double* ls = a.ql1 + ((size_t)b * a.NQ + q0) * K * 2;
  dc f[UF], g[UF];
#pragma unroll
  for (int u = 0; u < UF; ++u) {
    const int i = threadIdx.x + u * NT;
    if (i < nq * K) {
      f[u] = ld_dd(fs + 2 * i);
      if (with_l1) g[u] = ld_dd(ls + 2 * i);
    }
  }
  const float* src = a.qagg + ((size_t)b * a.NQ + q0) * a.D;
  f4a v[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int i = threadIdx.x + u * NT, q = i / R4, e = i - q * R4;
    if (i < nq * R4) v[u] = *reinterpret_cast<const f4a*>(src + (size_t)q * a.D + 4 * e);
  }
#pragma unroll
  for (int u = 0; u < UF; ++u) {
    const int i = threadIdx.x + u * NT;
    if (i < nq * K) {
      sg.F[i / K][i % K] = f[u];
      if (with_l1) sg.l1[i / K][i % K] = g[u];
    }
  }
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int i = threadIdx.x + u * NT, q = i / R4, e = i - q * R4;
    if (i < nq * R4) *reinterpret_cast<f4a*>(&sg.y[q][4 * e]) = v[u];
  }
}
struct QOps {
  PairSt y;
  dc y1k, Fj, Fk, l1k;
};
__device__ __forceinline__ QOps q_ops(const ScanLds& sg, int q, int j, int k, bool with_l1) {
  QOps o;
  o.y = load_st_f(sg.y[q], j, k);
  o.y1k = ld_fd(sg.y[q] + 2 * k);
  o.Fj = sg.F[q][j];
  o.Fk = sg.F[q][k];
  o.l1k = with_l1 ? sg.l1[q][k] : dc{0.0, 0.0};
  return o;
}
// block [lo, hi) of a segment of nq quads for wavefront w
__device__ __forceinline__ void seg_block(int nq, int w, int& lo, int& hi) {
  const int bq = (nq + SW - 1) / SW;
  lo = min(w * bq, nq);
  hi = min(lo + bq, nq);
}
__device__ __forceinline__ void put_block(ScanLds& sg, int w, int l, const PairSt& s) {
  sg.bS1[w][l] = s.S1;
  sg.bSA[w][l] = s.SA;
  sg.bSB[w][l] = s.SB;
}
__device__ __forceinline__ PairSt get_block(const ScanLds& sg, int w, int l) {
  return PairSt{sg.bS1[w][l], sg.bSA[w][l], sg.bSB[w][l]};
}

// Every global operand of the quad's chain (its chunks' mu rows, plane k's level-1 carries at the chunk bounds, the
// quad flow) is loaded before the first combine, so the wavefront waits for one round of loads, not one per chunk.
__global__ __launch_bounds__(64) void k_quad_bwd_agg(DiagArgs a) {
  __shared__ dc s_F[4][K];
  const int q = blockIdx.x, b = blockIdx.y, j = threadIdx.x >> 3, k = threadIdx.x & 7;
  const int c0 = 4 * q, nc = min(4, a.C - c0);
  PairSt m[4];
  dc cr[5];
#pragma unroll
  for (int i = 0; i < 4; ++i)
    if (i < nc) m[i] = load_st_f(a.mu + ((size_t)b * a.C + c0 + i) * a.D, j, k);
  const double* crow = a.carries + ((size_t)b * (a.C + 1) + c0) * a.D + 2 * k;
#pragma unroll
  for (int i = 0; i < 5; ++i)
    if (i <= nc) cr[i] = ld_dd(crow + (size_t)i * a.D);
  const dc Fq = threadIdx.x < K ? span_flow(a, b, c0, c0 + nc, k) : dc{1.0, 0.0};
  quad_flows(a, b, q, c0, nc, s_F);
  if (threadIdx.x < K) {  // the quad's level-1 increment, carry1(c0 + nc) - Fq carry1(c0)
    dc ce = cr[1];
#pragma unroll
    for (int i = 2; i < 5; ++i)
      if (i == nc) ce = cr[i];
    st_dd(a.ql1 + (((size_t)b * a.NQ + q) * K + k) * 2, ce - Fq * cr[0]);
  }
  PairSt X{};
#pragma unroll
  for (int i = 3; i >= 0; --i) {
    if (i < nc) {
      if (i < nc - 1) adj_d(X, s_F[i][j], s_F[i][k], cr[i + 1] - s_F[i][k] * cr[i]);
      add_st(X, m[i]);
    }
  }
  store_st_f(a.qagg + ((size_t)b * a.NQ + q) * a.D, j, k, X);
}

// Reverse scan of the adjoint carries, blocked as the forward scan: a block's aggregate is its cotangent at the
// block start from a zero cotangent at its end; its transfer is adj_d over the block's span (block flow and
// level-1 increment, carry1(end) - F carry1(start)).
__global__ __launch_bounds__(SW * 64) void k_quad_bwd_scan(DiagArgs a) {
  extern __shared__ __align__(16) char scan_smem[];
  ScanLds& sg = *reinterpret_cast<ScanLds*>(scan_smem);
  const int b = blockIdx.x, w = threadIdx.x >> 6, l = threadIdx.x & 63, j = l >> 3, k = l & 7;
  PairSt X{};  // cotangent at the segment end, kept by wavefront 0
  for (int qe = a.NQ; qe > 0; qe -= SSEG) {
    const int nq = min(SSEG, qe), q0 = qe - nq;
    int lo, hi;
    seg_block(nq, w, lo, hi);
    // plane k's level-1 carries at the block bounds (for the block's level-1 increment), loaded with the segment
    const int bc0 = 4 * (q0 + lo), bc1 = min(4 * (q0 + hi), a.C);
    dc cA{0.0, 0.0}, cB{0.0, 0.0};
    if (j == 0 && lo < hi) {
      cA = ld_dd(a.carries + ((size_t)b * (a.C + 1) + bc0) * a.D + 2 * k);
      cB = ld_dd(a.carries + ((size_t)b * (a.C + 1) + bc1) * a.D + 2 * k);
    }
    stage_seg(a, b, q0, nq, true, sg);
    __syncthreads();
    {  // 1. block aggregate from a zero cotangent at the block end; block flow and level-1 increment
      PairSt Xl{};
      dc Fk{1.0, 0.0};
      if (lo < hi) {
        QOps o = q_ops(sg, hi - 1, j, k, true);
        for (int q = hi - 1; q >= lo; --q) {
          const QOps cur = o;
          if (q > lo) o = q_ops(sg, q - 1, j, k, true);
          adj_d(Xl, cur.Fj, cur.Fk, cur.l1k);
          add_st(Xl, cur.y);
          Fk = Fk * cur.Fk;
        }
      }
      put_block(sg, w, l, Xl);
      if (j == 0) {
        sg.bF[w][k] = Fk;
        sg.bl1[w][k] = lo < hi ? cB - Fk * cA : dc{0.0, 0.0};  // carry1(bc1) - F carry1(bc0)
      }
    }
    __syncthreads();
    if (w == 0) {  // 2. cotangents at the block ends, last block first
      for (int v = SW - 1; v >= 0; --v) {
        const PairSt y = get_block(sg, v, l);
        const dc Fj = sg.bF[v][j], Fk = sg.bF[v][k], l1k = sg.bl1[v][k];
        put_block(sg, v, l, X);
        adj_d(X, Fj, Fk, l1k);
        add_st(X, y);
      }
    }
    __syncthreads();
    if (lo < hi) {  // 3. the cotangent at the last chunk of each quad of the block
      PairSt Xq = get_block(sg, w, l);
      QOps o = q_ops(sg, hi - 1, j, k, true);
      for (int q = hi - 1; q >= lo; --q) {
        const int c1 = min(4 * (q0 + q) + 4, a.C);
        store_st_f(a.mt + ((size_t)b * a.C + c1 - 1) * a.D, j, k, Xq);
        const QOps cur = o;
        if (q > lo) o = q_ops(sg, q - 1, j, k, true);
        adj_d(Xq, cur.Fj, cur.Fk, cur.l1k);
        add_st(Xq, cur.y);
      }
    }
    __syncthreads();  // the segment's LDS is restaged next
  }
}

// ------------------------------------------------------------------------------------------------ backward
// Cotangent row slice of the lane: level 1 of plane j and the KP 2x2 blocks (j, k).
template <int KP> struct GRow {
  f4a r0[KP / 2], r1[KP / 2];
  float2 g1;
};
// A prefetched cotangent row: the lane's pieces of the level-2 part and its level-1 pair.
template <int KP> struct GRaw {
  Pieces<KP> pc;
  f2u g1;
};
template <int KP> __device__ __forceinline__ GRaw<KP> load_graw(const float* row, int o1, int off2, int gl) {
  GRaw<KP> r;
  r.g1 = *reinterpret_cast<const f2u*>(row + o1);
  r.pc = load_pieces<KP>(row + off2, gl);
  return r;
}
// raw row -> LDS -> the lane's slice
// The level-1 pair goes through LDS too (buf[RBUF + 2j]), so that every register of the raw row is dead once
// this returns and a ring slot can be reloaded in place.
template <int KP> __device__ __forceinline__ GRow<KP> slice_g(const GRaw<KP>& r, float* buf, const Lane& l) {
  pieces_to_lds<KP>(r.pc, buf, l.gl);
  *reinterpret_cast<float2*>(buf + RBUF + 2 * l.j) = float2{r.g1.x, r.g1.y};
  wave_order();
  GRow<KP> g;
  g.g1 = *reinterpret_cast<const float2*>(buf + RBUF + 2 * l.j);
  const f4a* p0 = reinterpret_cast<const f4a*>(buf + row_at(2 * l.j) + 2 * KP * l.kg);
  const f4a* p1 = reinterpret_cast<const f4a*>(buf + row_at(2 * l.j + 1) + 2 * KP * l.kg);
  static_for<0, KP / 2>([&](auto ic) {
    constexpr int i = ic;
    g.r0[i] = p0[i];
    g.r1[i] = p1[i];
  });
  wave_order();
  return g;
}
// doubled pair cotangents (2 dL/dSA, 2 dL/dSB) of pair q from the block entries g00, g01, g10, g11
template <int KP, int q> __device__ __forceinline__ void g_pair(const GRow<KP>& g, cf& gA, cf& gB) {
  const f4a r0 = g.r0[q / 2], r1 = g.r1[q / 2];
  const float g00 = (q & 1) ? r0.z : r0.x, g01 = (q & 1) ? r0.w : r0.y;
  const float g10 = (q & 1) ? r1.z : r1.x, g11 = (q & 1) ? r1.w : r1.y;
  gA = cf{g00 + g11, g10 - g01};
  gB = cf{g00 - g11, g01 + g10};
}

// B1: chunk-local adjoint with zero incoming cotangent -> mu (cotangent on the chunk's carry-in state). KP = 4.
// SKIP_INV: the chunks whose steps may be inverted are left to the full local adjoint (k_bwd_full<.., BW_LOCAL>).
template <bool BF16, bool SKIP_INV>
__global__ __launch_bounds__(64) void k_bwd_local(DiagArgs a) {
  constexpr int KP = 4, GPW = Geo<KP>::GPW;
  __shared__ __align__(16) float s_v[2][GPW * VBLK];
  __shared__ __align__(16) float s_row[GPW][RBUF + DIM];  // cotangent row staging (+ level 1)
  const Lane l = lane_of<KP>(threadIdx.x);
  const int b = blockIdx.y, cb = blockIdx.x * GPW, c = cb + l.gi;
  const int nblk = (a.T + SB - 1) / SB;
  if constexpr (SKIP_INV) {  // nothing to do when every chunk of the workgroup is left to the full local adjoint
    bool any = false;
    for (int i = 0; i < GPW && cb + i < a.C; ++i) {
      const int fl = a.cflag[b * a.C + cb + i];
      any = any || ((fl & 1) && (fl & 3) != 3);
    }
    if (!any) return;
  }
  VRaw<GPW, BF16> vr;
  vblk_load<GPW, BF16>(a, b, cb, nblk - 1, vr);
  vblk_store<GPW, BF16>(a, cb, nblk - 1, vr, s_v[(nblk - 1) & 1]);
  __syncthreads();
  // every lane stays to the end (shared block staging); absent or non-uniform chunks skip the arithmetic
  const int ci = b * a.C + (c < a.C ? c : 0);
  const int flag = c < a.C ? a.cflag[ci] : 0;
  const bool active = (flag & 1) != 0 && !(SKIP_INV && (flag & 3) == 3);
  const int t0 = active ? c * a.T : 0, Tc = active ? min(a.T, a.n_int - t0) : 0;
  FwdCoef<KP> f;
  fwd_coef<KP>(a, l, active ? a.chbar[ci] : 0.0f, (flag & 4) != 0, f);
  const float* grow = a.gout + ((size_t)b * a.n_int + t0) * a.W;
  const int o1 = a.off1 + 2 * l.j;
  float* gbuf = s_row[l.gi];
  cf l1{0.0f, 0.0f}, lA[KP], lB[KP];
  static_for<0, KP>([&](auto qc) {
    constexpr int q = qc;
    lA[q] = lB[q] = cf{0.0f, 0.0f};
  });
  // Cotangent rows through a ring of RING register slots, RING steps ahead of their consumer. Every group runs
  // the steps t = nblk SB - 1 .. 0 so that every unrolled slot index is static; slot i holds row t of the step
  // t = tt - i. Loads and the LDS slicing are unconditional (rows clamped into the chunk), only the arithmetic
  // of steps t >= Tc is skipped: no load sits under a branch, and the waits before each use cover only the
  // oldest row.
  constexpr int RING = 2;
  static_assert(SB % RING == 0, "staged blocks hold whole ring rounds");
  GRaw<KP> ring[RING];
  static_for<0, RING>([&](auto ic) {
    constexpr int i = ic;
    ring[i] = load_graw<KP>(grow + (size_t)max(min(nblk * SB - 1 - i, Tc - 1), 0) * a.W, o1, a.off2, l.gl);
    __builtin_amdgcn_sched_barrier(0);  // issue the slots in consumption order (oldest load consumed first)
  });
  for (int blk = nblk - 1; blk >= 0; --blk) {
    if (blk > 0) vblk_load<GPW, BF16>(a, b, cb, blk - 1, vr);
    const float* vg = s_v[blk & 1] + l.gi * VBLK - blk * SB * DIM;  // indexed by the step t of the chunk
    for (int tt = blk * SB + SB - 1; tt >= blk * SB; tt -= RING) {
      static_for<0, RING>([&](auto ic) {
        constexpr int i = ic;
        const int t = tt - i;
        const GRow<KP> g = slice_g<KP>(ring[i], gbuf, l);
        ring[i] = load_graw<KP>(grow + (size_t)max(min(t - RING, Tc - 1), 0) * a.W, o1, a.off2, l.gl);
        if (t < Tc) {
          cf pj, pk[KP];
          load_p<KP>(vg + t * DIM, l, pj, pk);
          l1 += cf{g.g1.x, g.g1.y};
          cf toC{0.0f, 0.0f};
          static_for<0, KP>([&](auto qc) {
            constexpr int q = qc;
            cf gA, gB;
            g_pair<KP, q>(g, gA, gB);
            lA[q] += gA;
            lB[q] += gB;
            const cf sg = f.phk[q] * pk[q];
            toC += cjm(sg, lB[q]) + sg * lA[q];
            lB[q] = cjm(f.LB[q], lB[q]);
            lA[q] = cjm(f.LA[q], lA[q]);
          });
          l1 = cjm(f.rho, l1 + kg_sum<KP>(toC));
        }
      });
    }
    if (blk > 0) vblk_store<GPW, BF16>(a, cb, blk - 1, vr, s_v[(blk - 1) & 1]);
    wave_order();
  }
  if (!active) return;
  float* mp = a.mu + ((size_t)b * a.C + c) * a.D;
  if (l.kg == 0) *reinterpret_cast<float2*>(mp + 2 * l.j) = float2{l1.re, l1.im};
  static_for<0, KP>([&](auto qc) {
    constexpr int q = qc;
    *reinterpret_cast<f4a*>(mp + DIM + 4 * (l.j * K + KP * l.kg + q)) =
        f4a{0.5f * lA[q].re, 0.5f * lA[q].im, 0.5f * lB[q].re, 0.5f * lB[q].im};
  });
}

// B3: full adjoint of a uniform chunk whose steps may be inverted: states S(t-1) by inverting each step from the
// chunk's float64 end state; cotangents from mt (later chunks) plus the readout rows. Writes the knot gradients
// of the chunk's interior knots directly (dpath, dclock), dv / dh of its first and last interval (the chunk
// boundary knots are finished by k_knot_bounds), and the chunk's parameter partials. KP = 2 (32-lane groups).
template <int KP> struct BwdCoef {
  cf rho, rhoi, phi, rho1, phi1;        // plane j (rho1, phi1 = d/dh)
  cf phk[KP], phi1h[KP];                // phi_k / 2, (d phi_k / dh) / 2
  cf LB[KP], LA[KP], LBi[KP], LAi[KP];  // pair flows and their inverses
  cf IB[KP], IA[KP], IB1[KP], IA1[KP];  // IB / 2, IA / 2, d/dh of those
  cf LB1[KP], LA1[KP];                  // d/dh of the flows
};

// Modes of the invertible-chunk adjoint. BW_FULL: the adjoint from the cotangent of the later chunks (mt) plus the
// readout rows, as described above. BW_LOCAL: the same per-step adjoint from a zero cotangent at the chunk end (the
// chunk's own rows only): writes dv of every step (a.dv), the chunk's parameter partials and mu (the cotangent on
// the carry-in state, for the adjoint scan); the later chunks' part is added by k_bwd_carry in closed form.
constexpr int BW_FULL = 0, BW_LOCAL = 1;

// DH: the clock gradient is requested (dclock non-null); without it the step skips every dh term (BW_LOCAL runs
// without it only).
template <bool BF16, bool DH, int MODE>
__global__ __launch_bounds__(64) void k_bwd_full(DiagArgs a) {
  static_assert(MODE == BW_FULL || !DH, "the local adjoint runs without the clock gradient");
  constexpr int KP = 2, G = Geo<KP>::G, GPW = Geo<KP>::GPW;
  __shared__ __align__(16) float s_v[GPW * VPITCH];
  __shared__ float s_h[GPW * kMaxT];
  __shared__ __align__(16) float s_w[GPW][NB * K * K * 2];  // column terms w[t][k][j] (complex)
  __shared__ __align__(16) float s_dvp[GPW][NB * K * 2];    // plane part of dv[t][j] (complex)
  __shared__ __align__(16) float s_dhp[GPW][NB * G];        // dh partials [t][lane]
  __shared__ __align__(16) float s_dvo[GPW][(NB + 1) * DIM];  // dv of the block's steps; row NB: the step after
  __shared__ float s_dho[GPW][NB + 1];
  __shared__ __align__(16) float s_row[GPW][RBUF + DIM];  // cotangent row staging (+ level 1)
  __shared__ __align__(16) float s_mt[GPW][DIM + DIM * DIM];  // cotangent from later chunks, per group
  __shared__ float s_dhr[DH ? GPW : 1][DH ? G : 1];   // the first step's dh partials without the flow terms
  __shared__ double s_f64[GPW];                         // <mt(c - 1), D carry(c)> of each chunk (float64)
  const Lane l = lane_of<KP>(threadIdx.x);
  const int b = blockIdx.y, cb = blockIdx.x * GPW, c = cb + l.gi;
  stage<KP, BF16>(a, b, cb, s_v, s_h);
  if constexpr (MODE == BW_FULL) {
    // adjoint carries inside the quad: mt[c] = mu(c+1) + J_{c+1}^T mt[c+1] down from the quad's last chunk
    // (written by the scan); float64, written back for every later kernel that reads mt (generic chunks)
    const int jj = threadIdx.x >> 3, kk = threadIdx.x & 7;
    const int q0 = 4 * (cb / 4), c_last = min(q0 + 3, a.C - 1);
    PairSt X = load_st_f(a.mt + ((size_t)b * a.C + c_last) * a.D, jj, kk);
    if (c_last < cb + GPW) store_st_f(s_mt[c_last - cb], jj, kk, X);
    // with the clock gradient: the flow part of the chunk's first-step dh is <mt(c - 1), D carry(c)> (the
    // carried cotangent on the state before the chunk, against the flows' derivative of that state), taken in
    // float64 from the scanned cotangent and the float64 carry, so that the boundary knot's dh difference pairs
    // it with the previous chunk's last step, which sees the same cotangent and state (the float32 adjoint
    // recursion over the chunk drifts from it by more than the knot gradient's tolerance at L = 18k)
    auto first_flow = [&](int ci, const PairSt& m) {
      const double f = wave_sum_d(flow_dot(a, m, load_st_d(a.carries + ((size_t)b * (a.C + 1) + ci) * a.D, jj, kk),
                                           jj, kk));
      if (threadIdx.x == 0) s_f64[ci - cb] = f;
    };
    const int c_stop = DH ? max(cb - 1, q0) : cb;
    for (int cc = c_last - 1; cc >= c_stop; --cc) {
      const double* cf = a.cflow + ((size_t)b * a.C + cc + 1) * K * 2;
      const dc Fk = ld_dd(cf + 2 * kk);
      adj_d(X, ld_dd(cf + 2 * jj), Fk, l1_inc(a, b, cc + 1, cc + 2, kk, Fk));
      add_st(X, load_st_f(a.mu + ((size_t)b * a.C + cc + 1) * a.D, jj, kk));
      if (cc >= cb && cc < cb + GPW) {
        store_st_f(s_mt[cc - cb], jj, kk, X);
        store_st_f(a.mt + ((size_t)b * a.C + cc) * a.D, jj, kk, X);
      }
      if (DH && cc + 1 < cb + GPW) first_flow(cc + 1, X);
    }
    if constexpr (DH) {
      if (cb == q0 && cb >= 1) first_flow(cb, load_st_f(a.mt + ((size_t)b * a.C + cb - 1) * a.D, jj, kk));
      if (cb == 0 && threadIdx.x == 0) s_f64[0] = 0.0;  // the zero state before the first chunk
    }
  }
  __syncthreads();
  const int ci = b * a.C + (c < a.C ? c : 0);
  const bool active = c < a.C && (a.cflag[ci] & 3) == 3;
  const int t0 = c * a.T, Tc = active ? min(a.T, a.n_int - t0) : 0;
  const float hb = active ? a.chbar[ci] : 0.0f;
  // coefficients at hbar
  BwdCoef<KP> f;
  const bool use_tab = active && (a.cflag[ci] & 4);
  const cf uj = load_u(a.params, l.j);
  const cf xj = hb * uj;
  if (use_tab) {
    const float* tab = a.ctab;
    const float dlt = hb - tab[0];
    f.rho = tflow(tp(tab, l.j, TP_RHO), tp(tab, l.j, TP_RHO1), dlt);
    f.rhoi = tflow(tp(tab, l.j, TP_RHOI), tp(tab, l.j, TP_RHOI1), dlt);
    f.phi = tp(tab, l.j, TP_PHI);
    f.rho1 = tp(tab, l.j, TP_RHO1);
    f.phi1 = tp(tab, l.j, TP_PHI1);
    static_for<0, KP>([&](auto qc) {
      constexpr int q = qc;
      const int k = KP * l.kg + q;
      f.phk[q] = tp(tab, k, TP_PHIH);
      f.phi1h[q] = tp(tab, k, TP_PHI1H);
      f.LB[q] = tflow(tq(tab, l.j, k, TQ_LB), tq(tab, l.j, k, TQ_LB1), dlt);
      f.LA[q] = tflow(tq(tab, l.j, k, TQ_LA), tq(tab, l.j, k, TQ_LA1), dlt);
      f.LBi[q] = tflow(tq(tab, l.j, k, TQ_LBI), tq(tab, l.j, k, TQ_LBI1), dlt);
      f.LAi[q] = tflow(tq(tab, l.j, k, TQ_LAI), tq(tab, l.j, k, TQ_LAI1), dlt);
      f.LB1[q] = tq(tab, l.j, k, TQ_LB1);
      f.LA1[q] = tq(tab, l.j, k, TQ_LA1);
      f.IB[q] = tq(tab, l.j, k, TQ_IB);
      f.IA[q] = tq(tab, l.j, k, TQ_IA);
      f.IB1[q] = tq(tab, l.j, k, TQ_IB1);
      f.IA1[q] = tq(tab, l.j, k, TQ_IA1);
    });
  } else {
    const Node1<cf> nj = node1(xj);
    f.rho = nj.e;
    f.rhoi = expv(-xj);
    f.phi = nj.p;
    f.rho1 = nj.e * uj;
    f.phi1 = nj.dp * uj;
    static_for<0, KP>([&](auto qc) {
      constexpr int q = qc;
      const cf uk = load_u(a.params, KP * l.kg + q);
      const Node1<cf> nk = node1(hb * uk);
      f.phk[q] = 0.5f * nk.p;
      f.phi1h[q] = 0.5f * (nk.dp * uk);
      const cf ub = uj + uk, ua = uj + conj(uk);
      f.LB[q] = expv(hb * ub);
      f.LA[q] = expv(hb * ua);
      f.LBi[q] = expv(-(hb * ub));
      f.LAi[q] = expv(-(hb * ua));
      f.LB1[q] = f.LB[q] * ub;
      f.LA1[q] = f.LA[q] * ua;
      const DD3<cf> db = dd3<cf, true>(xj, hb * ub);
      const DD3<cf> da = dd3<cf, true>(xj, hb * ua);
      f.IB[q] = 0.5f * db.d;
      f.IA[q] = 0.5f * da.d;
      f.IB1[q] = 0.5f * (db.dx * uj + db.dy * ub);
      f.IA1[q] = 0.5f * (da.dx * uj + da.dy * ua);
    });
  }
  // end state (float64 carry after the chunk) and cotangent from later chunks
  cf S1{0.0f, 0.0f}, SA[KP], SB[KP], l1{0.0f, 0.0f}, lA[KP], lB[KP];
  static_for<0, KP>([&](auto qc) {
    constexpr int q = qc;
    SA[q] = SB[q] = lA[q] = lB[q] = cf{0.0f, 0.0f};
  });
  if (active) {
    const double* cr = a.carries + ((size_t)b * (a.C + 1) + c + 1) * a.D;
    const float* mp = s_mt[l.gi];
    S1 = cf{(float)cr[2 * l.j], (float)cr[2 * l.j + 1]};
    if constexpr (MODE == BW_FULL) l1 = cf{mp[2 * l.j], mp[2 * l.j + 1]};
    static_for<0, KP>([&](auto qc) {
      constexpr int q = qc;
      const int e = DIM + 4 * (l.j * K + KP * l.kg + q);
      SA[q] = cf{(float)(0.5 * cr[e]), (float)(0.5 * cr[e + 1])};
      SB[q] = cf{(float)(0.5 * cr[e + 2]), (float)(0.5 * cr[e + 3])};
      if constexpr (MODE == BW_FULL) {
        const f4a m = *reinterpret_cast<const f4a*>(mp + e);
        lA[q] = cf{2.0f * m.x, 2.0f * m.y};
        lB[q] = cf{2.0f * m.z, 2.0f * m.w};
      }
    });
  }
  // parameter-gradient accumulators (sums of h_t times coefficient cotangents)
  cf kIB[KP], kIA[KP], kLB[KP], kLA[KP], kph[KP], krho{0.0f, 0.0f}, kphj{0.0f, 0.0f};
  static_for<0, KP>([&](auto qc) {
    constexpr int q = qc;
    kIB[q] = kIA[q] = kLB[q] = kLA[q] = kph[q] = cf{0.0f, 0.0f};
  });

  const float* vg = s_v + l.gi * VPITCH;
  const float* hg = s_h + l.gi * kMaxT;
  float* w_g = s_w[l.gi];
  float* dvp_g = s_dvp[l.gi];
  float* dhp_g = s_dhp[l.gi];
  float* dvo_g = s_dvo[l.gi];
  float* dho_g = s_dho[l.gi];
  const float* grow = a.gout + ((size_t)b * a.n_int + (active ? t0 : 0)) * a.W;
  const int o1 = a.off1 + 2 * l.j;
  float* gbuf = s_row[l.gi];
  // cotangent rows through a ring of NB register slots: row t sits in slot t % NB (the step's static index in
  // the unrolled block below) and is reloaded with row t - NB right after use, NB steps ahead of its consumer
  GRaw<KP> ring[NB];
  // (loads and slicing are unconditional, rows clamped into the chunk; only the arithmetic of steps t >= Tc is
  // skipped, so no load sits under a branch and the waits before each use cover only the oldest row)
  const int nblk = (a.T + NB - 1) / NB;
  static_down<NB - 1>([&](auto sc) {  // slot s holds row tb + s of the first block processed
    constexpr int s = sc;
    ring[s] = load_graw<KP>(grow + (size_t)max(min((nblk - 1) * NB + s, Tc - 1), 0) * a.W, o1, a.off2, l.gl);
    __builtin_amdgcn_sched_barrier(0);  // issue the slots in consumption order (oldest load consumed first)
  });
  // blocks of NB steps, last block first; every group runs the same number of blocks (barriers)
  for (int blk = nblk - 1; blk >= 0; --blk) {
    const int tb = blk * NB;
    static_down<NB - 1>([&](auto sc) {
      constexpr int s = sc;
      const int t = tb + s;
      const GRow<KP> g = slice_g<KP>(ring[s], gbuf, l);
      ring[s] = load_graw<KP>(grow + (size_t)max(min(t - NB, Tc - 1), 0) * a.W, o1, a.off2, l.gl);
      if (t >= Tc) return;
      const float h = hg[t];
      cf pj, pk[KP];
      load_p<KP>(vg + t * DIM, l, pj, pk);
      l1 += cf{g.g1.x, g.g1.y};
      // invert the level-1 step: c_j = rho S1(t-1) = S1(t) - phi_j p_j
      const cf cj = S1 - f.phi * pj;
      const cf H1 = f.rhoi * cj;
      cf toC{0.0f, 0.0f}, toP{0.0f, 0.0f};
      float dhp = 0.0f, dhf = 0.0f;  // dhf: the flow terms of dhp
      if constexpr (DH) {
        static_for<0, KP>([&](auto qc) {
          constexpr int q = qc;
          cf gA, gB;
          g_pair<KP, q>(g, gA, gB);
          const cf A = lA[q] + gA, Bc = lB[q] + gB;  // doubled cotangents of SA(t), SB(t)
          const cf sg = f.phk[q] * pk[q];
          cf pi, pic;
          prods(pj, pk[q], pi, pic);
          const cf XB = SB[q] - cj * sg - f.IB[q] * pi;
          const cf XA = SA[q] - cj * conj(sg) - f.IA[q] * pic;
          const cf HB = f.LBi[q] * XB;
          const cf HA = f.LAi[q] * XA;
          // row terms (plane j)
          toC += cjm(sg, Bc) + sg * A;
          const cf gf = cjm(f.IB[q], Bc);
          const cf ge = cjm(f.IA[q], A);
          toP += cjm(pk[q], gf) + pk[q] * ge;
          // column terms (plane k): dv_k share and the phi_k cotangent share
          const cf tS = cjm(cj, Bc) + cjm(A, cj);
          const cf w = cjm(f.phk[q], tS) + cjm(pj, gf) + cjm(ge, pj);
          *reinterpret_cast<float2*>(w_g + ((s * K + KP * l.kg + q) * K + l.j) * 2) = float2{w.re, w.im};
          const cf gph = cjm(pk[q], tS);
          if constexpr (DH) dhp += redot(gph, f.phi1h[q]);
          kph[q] = fma_c(cf{h, 0.0f}, gph, kph[q]);
          // coefficient cotangents
          const cf gIB = cjm(pi, Bc), gIA = cjm(pic, A), gLB = cjm(HB, Bc), gLA = cjm(HA, A);
          if constexpr (DH) {
            const float fl = redot(gLB, f.LB1[q]) + redot(gLA, f.LA1[q]);
            dhp += redot(gIB, f.IB1[q]) + redot(gIA, f.IA1[q]) + fl;
            dhf += fl;
          }
          kIB[q] = fma_c(cf{h, 0.0f}, gIB, kIB[q]);
          kIA[q] = fma_c(cf{h, 0.0f}, gIA, kIA[q]);
          kLB[q] = fma_c(cf{h, 0.0f}, gLB, kLB[q]);
          kLA[q] = fma_c(cf{h, 0.0f}, gLA, kLA[q]);
          lB[q] = cjm(f.LB[q], Bc);
          lA[q] = cjm(f.LA[q], A);
          SB[q] = HB;
          SA[q] = HA;
        });
      } else {
        // the same step in explicit real arithmetic, shared sums P = Bc + A, Q = Bc - A and F = gf + ge,
        // E = gf - ge; the coefficient cotangents accumulate as dot products with the h-scaled cotangents
        static_for<0, KP>([&](auto qc) {
          constexpr int q = qc;
          cf gA, gB;
          g_pair<KP, q>(g, gA, gB);
          const float Ar = lA[q].re + gA.re, Ai = lA[q].im + gA.im;  // doubled cotangents of SA(t), SB(t)
          const float Br = lB[q].re + gB.re, Bi = lB[q].im + gB.im;
          const float Pr = Br + Ar, Pi = Bi + Ai, Qr = Br - Ar, Qi = Bi - Ai;
          const cf pkq = pk[q], ph = f.phk[q];
          const float sgr = fmaf(ph.re, pkq.re, -ph.im * pkq.im), sgi = fmaf(ph.re, pkq.im, ph.im * pkq.re);
          const float aa = pj.re * pkq.re, bb = pj.im * pkq.im, cc = pj.re * pkq.im, dd = pj.im * pkq.re;
          const float pir = aa - bb, pii = cc + dd, pcr = aa + bb, pci = dd - cc;  // p_j p_k, p_j conj(p_k)
          const float rr = cj.re * sgr, ii = cj.im * sgi, ri = cj.re * sgi, ir = cj.im * sgr;
          const cf IB = f.IB[q], IA = f.IA[q];
          // previous states: X = S(t) - local terms, H = flow^-1 X
          const float XBr = fmaf(IB.im, pii, fmaf(-IB.re, pir, SB[q].re - rr + ii));
          const float XBi = fmaf(-IB.im, pir, fmaf(-IB.re, pii, SB[q].im - ri - ir));
          const float XAr = fmaf(IA.im, pci, fmaf(-IA.re, pcr, SA[q].re - rr - ii));
          const float XAi = fmaf(-IA.im, pcr, fmaf(-IA.re, pci, SA[q].im - ir + ri));
          const cf LBi = f.LBi[q], LAi = f.LAi[q];
          const float HBr = fmaf(LBi.re, XBr, -LBi.im * XBi), HBi = fmaf(LBi.re, XBi, LBi.im * XBr);
          const float HAr = fmaf(LAi.re, XAr, -LAi.im * XAi), HAi = fmaf(LAi.re, XAi, LAi.im * XAr);
          // row terms (plane j): toC += conj(sg) Bc + sg A; toP += conj(p_k) gf + p_k ge
          toC.re = fmaf(sgr, Pr, fmaf(sgi, Qi, toC.re));
          toC.im = fmaf(sgr, Pi, fmaf(-sgi, Qr, toC.im));
          const float gfr = fmaf(IB.re, Br, IB.im * Bi), gfi = fmaf(IB.re, Bi, -IB.im * Br);  // conj(IB) Bc
          const float ger = fmaf(IA.re, Ar, IA.im * Ai), gei = fmaf(IA.re, Ai, -IA.im * Ar);  // conj(IA) A
          const float Fr = gfr + ger, Fi = gfi + gei, Er = gfr - ger, Ei = gfi - gei;
          toP.re = fmaf(pkq.re, Fr, fmaf(pkq.im, Ei, toP.re));
          toP.im = fmaf(pkq.re, Fi, fmaf(-pkq.im, Er, toP.im));
          // column terms (plane k): tS = conj(c_j) Bc + conj(A) c_j; w = conj(phi_k/2) tS + conj(p_j) gf + conj(ge) p_j
          const float tSr = fmaf(cj.re, Pr, cj.im * Pi), tSi = fmaf(cj.re, Qi, -cj.im * Qr);
          const float wr = fmaf(ph.re, tSr, fmaf(ph.im, tSi, fmaf(pj.re, Fr, pj.im * Fi)));
          const float wi = fmaf(ph.re, tSi, fmaf(-ph.im, tSr, fmaf(pj.re, Ei, -pj.im * Er)));
          *reinterpret_cast<float2*>(w_g + ((s * K + KP * l.kg + q) * K + l.j) * 2) = float2{wr, wi};
          // coefficient cotangents, summed with the step's h: conj(p_k) tS, conj(pi) Bc, conj(pic) A,
          // conj(HB) Bc, conj(HA) A
          const float tSrh = h * tSr, tSih = h * tSi, Brh = h * Br, Bih = h * Bi, Arh = h * Ar, Aih = h * Ai;
          kph[q].re = fmaf(pkq.re, tSrh, fmaf(pkq.im, tSih, kph[q].re));
          kph[q].im = fmaf(pkq.re, tSih, fmaf(-pkq.im, tSrh, kph[q].im));
          kIB[q].re = fmaf(pir, Brh, fmaf(pii, Bih, kIB[q].re));
          kIB[q].im = fmaf(pir, Bih, fmaf(-pii, Brh, kIB[q].im));
          kIA[q].re = fmaf(pcr, Arh, fmaf(pci, Aih, kIA[q].re));
          kIA[q].im = fmaf(pcr, Aih, fmaf(-pci, Arh, kIA[q].im));
          kLB[q].re = fmaf(HBr, Brh, fmaf(HBi, Bih, kLB[q].re));
          kLB[q].im = fmaf(HBr, Bih, fmaf(-HBi, Brh, kLB[q].im));
          kLA[q].re = fmaf(HAr, Arh, fmaf(HAi, Aih, kLA[q].re));
          kLA[q].im = fmaf(HAr, Aih, fmaf(-HAi, Arh, kLA[q].im));
          // adjoint carried to the previous step, state stepped back
          const cf LB = f.LB[q], LA = f.LA[q];
          lB[q] = cf{fmaf(LB.re, Br, LB.im * Bi), fmaf(LB.re, Bi, -LB.im * Br)};
          lA[q] = cf{fmaf(LA.re, Ar, LA.im * Ai), fmaf(LA.re, Ai, -LA.im * Ar)};
          SB[q] = cf{HBr, HBi};
          SA[q] = cf{HAr, HAi};
        });
      }
      toC = kg_sum<KP>(toC);
      toP = kg_sum<KP>(toP);
      const cf gc = l1 + toC;
      if (l.kg == 0) {
        const cf dvp = cjm(f.phi, l1) + toP;
        *reinterpret_cast<float2*>(dvp_g + (s * K + l.j) * 2) = float2{dvp.re, dvp.im};
        const cf gphL = cjm(pj, l1);
        const cf grho = cjm(H1, gc);
        if constexpr (DH) {
          const float fl = redot(grho, f.rho1);
          dhp += redot(gphL, f.phi1) + fl;
          dhf += fl;
        }
        kphj = fma_c(cf{h, 0.0f}, gphL, kphj);
        krho = fma_c(cf{h, 0.0f}, grho, krho);
      }
      if constexpr (DH) {
        dhp_g[s * G + l.gl] = dhp;
        if (t == 0) s_dhr[l.gi][l.gl] = dhp - dhf;
      }
      l1 = cjm(f.rho, gc);
      S1 = H1;
    });
    __syncthreads();
    // column sums of the block: dv[t][k] = plane part + sum_j w[t][k][j]; dh[t] = sum of the lane partials
    for (int it = l.gl; it < NB * K; it += G) {
      const int s = it >> 3, k = it & 7, t = tb + s;
      if (t < Tc) {
        const f4a* wp = reinterpret_cast<const f4a*>(w_g + (s * K + k) * K * 2);
        const f4a acc = wp[0] + wp[1] + wp[2] + wp[3];
        float2 dv = *reinterpret_cast<const float2*>(dvp_g + (s * K + k) * 2);
        dv.x += acc.x + acc.z;
        dv.y += acc.y + acc.w;
        *reinterpret_cast<float2*>(dvo_g + s * DIM + 2 * k) = dv;
        // boundary intervals: their knots are finished by k_knot_bounds; the local adjoint keeps every step's dv
        if (MODE == BW_LOCAL || t == 0 || t == Tc - 1)
          *reinterpret_cast<float2*>(a.dv + ((size_t)b * a.n_int + t0 + t) * DIM + 2 * k) = dv;
      }
    }
    if (DH && l.gl < NB) {
      const int s = l.gl, t = tb + s;
      if (t < Tc) {
        float acc = 0.0f;
        for (int q = 0; q < G; q += 4) {
          const f4a v = *reinterpret_cast<const f4a*>(dhp_g + s * G + q);
          acc += (v.x + v.y) + (v.z + v.w);
        }
        dho_g[s] = acc;
        if (t == Tc - 1) {
          a.dh[(size_t)b * a.n_int + t0 + t] = acc;
        } else if (t == 0) {  // the first step's dh for its boundary knot: local terms here, flows in float64
          double r = 0.0;
          for (int q = 0; q < G; ++q) r += (double)s_dhr[l.gi][q];
          a.dh[(size_t)b * a.n_int + t0] = (float)(r + s_f64[l.gi]);
        }
      }
    }
    __syncthreads();
    if constexpr (MODE == BW_LOCAL) continue;  // the knots are written by k_bwd_carry
    // interior knots tb+1 .. tb+NB of the chunk: dX = dv(t-1) - dv(t), dtheta = dh(t-1) - dh(t); row NB of the
    // block arrays holds the step after the block (the first step of the block processed before)
    for (int it = l.gl; it < NB * (DIM + 1); it += G) {
      const int s = 1 + it / (DIM + 1), ch = it % (DIM + 1), t = tb + s;
      if (t >= 1 && t <= Tc - 1) {
        if (ch < DIM) {
          a.dpath[((size_t)b * a.L + t0 + t) * DIM + ch] = dvo_g[(s - 1) * DIM + ch] - dvo_g[s * DIM + ch];
        } else if (DH) {
          a.dclock[(size_t)b * a.L + t0 + t] = dho_g[s - 1] - dho_g[s];
        }
      }
    }
    __syncthreads();
    for (int it = l.gl; it < DIM + 1; it += G) {  // keep this block's first step for the next (earlier) block
      if (it < DIM) dvo_g[NB * DIM + it] = dvo_g[it];
      else dho_g[NB] = dho_g[0];
    }
    __syncthreads();
  }
  // parameter partials of the chunk: node cotangents -> (d_j, w_j) per plane. A node h u contributes
  // (-Re G, Im G) to its plane for u = -conj(z) and (-Re G, -Im G) for u = -z (the conj(u_k) of the A pairs).
  constexpr int PS = 2 + 2 * KP;  // per-lane floats: row part, then one (d, w) per column pair
  float* sp = s_w[l.gi];          // reuses the column-sum area
  if constexpr (MODE == BW_LOCAL) {  // mu: the cotangent on the chunk's carry-in state (halved pair cotangents)
    if (active) {
      float* mp = a.mu + ((size_t)b * a.C + c) * a.D;
      if (l.kg == 0) *reinterpret_cast<float2*>(mp + 2 * l.j) = float2{l1.re, l1.im};
      static_for<0, KP>([&](auto qc) {
        constexpr int q = qc;
        *reinterpret_cast<f4a*>(mp + DIM + 4 * (l.j * K + KP * l.kg + q)) =
            f4a{0.5f * lA[q].re, 0.5f * lA[q].im, 0.5f * lB[q].re, 0.5f * lB[q].im};
      });
    }
  }
  if (active) {
    float rd = 0.0f, rw = 0.0f;
    cf Gx{0.0f, 0.0f};
    static_for<0, KP>([&](auto qc) {
      constexpr int q = qc;
      const int k = KP * l.kg + q;
      cf DxB, DyB, DxA, DyA, dpk;
      if (use_tab) {
        DxB = tq(a.ctab, l.j, k, TQ_DXB);
        DyB = tq(a.ctab, l.j, k, TQ_DYB);
        DxA = tq(a.ctab, l.j, k, TQ_DXA);
        DyA = tq(a.ctab, l.j, k, TQ_DYA);
        dpk = tp(a.ctab, k, TP_DPHI);
      } else {
        const cf uk = load_u(a.params, k);
        const cf ub = uj + uk, ua = uj + conj(uk);
        const DD3<cf> db = dd3<cf, true>(xj, hb * ub);
        const DD3<cf> da = dd3<cf, true>(xj, hb * ua);
        DxB = db.dx;
        DyB = db.dy;
        DxA = da.dx;
        DyA = da.dy;
        dpk = node1(hb * uk).dp;
      }
      Gx += 0.5f * (kIB[q] * conj(DxB) + kIA[q] * conj(DxA));
      const cf GyB = 0.5f * (kIB[q] * conj(DyB)) + kLB[q] * conj(f.LB[q]);
      const cf GyA = 0.5f * (kIA[q] * conj(DyA)) + kLA[q] * conj(f.LA[q]);
      const cf Gk = 0.5f * (kph[q] * conj(dpk));
      rd += -GyB.re - GyA.re;
      rw += GyB.im + GyA.im;
      sp[l.gl * PS + 2 + 2 * q] = -GyB.re - GyA.re - Gk.re;
      sp[l.gl * PS + 3 + 2 * q] = GyB.im - GyA.im + Gk.im;
    });
    if (l.kg == 0) {
      const cf dpj = use_tab ? tp(a.ctab, l.j, TP_DPHI) : node1(xj).dp;
      Gx += krho * conj(f.rho) + kphj * conj(dpj);
    }
    sp[l.gl * PS + 0] = rd - Gx.re;
    sp[l.gl * PS + 1] = rw + Gx.im;
  }
  __syncthreads();
  if (active && l.gl < K) {
    const int p = l.gl, pkg = p / KP, pq = p % KP;
    float sd = 0.0f, sw = 0.0f;
    for (int kg = 0; kg < Geo<KP>::NKG; ++kg) {
      sd += sp[(p + 8 * kg) * PS];
      sw += sp[(p + 8 * kg) * PS + 1];
    }
    for (int jj = 0; jj < K; ++jj) {
      const int src = pkg * 8 + jj;
      sd += sp[src * PS + 2 + 2 * pq];
      sw += sp[src * PS + 3 + 2 * pq];
    }
    float* gpo = a.gp + ((size_t)b * a.C + c) * a.npar;
    gpo[2 * p] = sd;
    gpo[2 * p + 1] = sw;
  }
}

// ------------------------------------------------------------------------------------------------ carry adjoint
// The part of an invertible uniform chunk's adjoint that the cotangent of the later chunks (mt, the cotangent on
// the chunk's end state) drives, in closed form; k_bwd_full<.., BW_LOCAL> has added the part of the chunk's own
// readout rows. Linear in that cotangent, with the chunk's coefficients constant, every term is a fixed K x K
// matrix applied to per-step vectors. Let n_t = span of the steps after t to the chunk end (clock theta_end -
// theta_{t+1}), a_{t,j} = conj(exp(u_j n_t)) (the adjoint flow of plane j from the chunk end back to step t),
// pi_{t,j} = p_{t,j} conj(a_{t,j}), sigma = (phi/2) pi, gamma_{t,j} = c_{t,j} conj(a_{t,j}) with c = rho S1(t-1) the
// level-1 state; lamB, lamA (doubled) and lam1 the end cotangents, GB = conj(IB/2) lamB, GA = conj(IA/2) lamA. Then
//   level-2 cotangents  B_t = a_j a_k lamB,  A_t = a_j conj(a_k) lamA
//   RC_t[j] = sum_k conj(sigma_k) lamB[j,k] + sigma_k lamA[j,k],   RP_t[j] = sum_k conj(pi_k) GB + pi_k GA
//   CS_t[k] = conj(phi_k/2) sum_j (conj(gamma_j) lamB + conj(lamA) gamma_j) + sum_j (conj(pi_j) GB + conj(GA) pi_j)
//   level-1 cotangent   l1_t = a_j (lam1 + sum_{s>t} RC_s[j])   (the flows telescope)
//   dv_t (plane m)      = a_m (conj(phi_m) (lam1 + sum_{s>t} RC_s) + RP_t[m]) + a_m CS_t[m]
// and the coefficient cotangents summed with h (the parameter gradients) are outer-product sums over the steps:
//   kIB = lamB conj(sum h pi_j pi_k), kIA = lamA conj(sum h pi_j conj(pi_k)),
//   kph = lamB conj(sum h gamma_j pi_k) + conj(lamA) sum h gamma_j conj(pi_k),
//   kLB = lamB conj(W_B), W_B = (C2B/2 e^{(u_j+u_k) tau} tau + (phi_k/2) sum n gamma_j pi_k + (IB/2) sum n pi_j pi_k) / LB
//   (kLA alike with conj(u_k), conj(phi_k/2), conj(pi_k)), kphj = sum h conj(pi_j) (lam1 + sum_{s>t} RC_s),
//   krho = sum h conj(S1(t-1)) a_j (lam1 + sum_{s>=t} RC_s);
// C2 / 2 is the halved level-2 carry-in state and tau the chunk's clock span. One wavefront per chunk: lane = step
// for the per-step vectors and matvecs, lane = pair (j, k) for the outer-product sums. Writes the chunk's total
// dv (local part + this), its interior knot gradients and adds its parameter partials to the local ones.
struct PairCoefs {
  cf rho_j, phi_j, dphi_j, phk_k, dphi_k, IB, IA, LB, LA, DxB, DyB, DxA, DyA;
};
__device__ __forceinline__ PairCoefs pair_coefs(const DiagArgs& a, int j, int k, float hb, bool use_tab) {
  PairCoefs o;
  if (use_tab) {
    const float* tab = a.ctab;
    const float dlt = hb - tab[0];
    o.rho_j = tflow(tp(tab, j, TP_RHO), tp(tab, j, TP_RHO1), dlt);
    o.phi_j = tp(tab, j, TP_PHI);
    o.dphi_j = tp(tab, j, TP_DPHI);
    o.phk_k = tp(tab, k, TP_PHIH);
    o.dphi_k = tp(tab, k, TP_DPHI);
    o.IB = tq(tab, j, k, TQ_IB);
    o.IA = tq(tab, j, k, TQ_IA);
    o.LB = tflow(tq(tab, j, k, TQ_LB), tq(tab, j, k, TQ_LB1), dlt);
    o.LA = tflow(tq(tab, j, k, TQ_LA), tq(tab, j, k, TQ_LA1), dlt);
    o.DxB = tq(tab, j, k, TQ_DXB);
    o.DyB = tq(tab, j, k, TQ_DYB);
    o.DxA = tq(tab, j, k, TQ_DXA);
    o.DyA = tq(tab, j, k, TQ_DYA);
    return o;
  }
  const cf uj = load_u(a.params, j), uk = load_u(a.params, k);
  const cf xj = hb * uj;
  const Node1<cf> nj = node1(xj), nk = node1(hb * uk);
  o.rho_j = nj.e;
  o.phi_j = nj.p;
  o.dphi_j = nj.dp;
  o.phk_k = 0.5f * nk.p;
  o.dphi_k = nk.dp;
  const cf ub = uj + uk, ua = uj + conj(uk);
  o.LB = expv(hb * ub);
  o.LA = expv(hb * ua);
  const DD3<cf> db = dd3<cf, true>(xj, hb * ub);
  const DD3<cf> da = dd3<cf, true>(xj, hb * ua);
  o.IB = 0.5f * db.d;
  o.IA = 0.5f * da.d;
  o.DxB = db.dx;
  o.DyB = db.dy;
  o.DxA = da.dx;
  o.DyA = da.dy;
  return o;
}
// sum_k conj(x_k) M1 + x_k M2 from m = (M1r + M2r, M1i - M2i, M1i + M2i, M2r - M1r)
__device__ __forceinline__ void acc_row(cf& r, cf x, f4a m) {
  r.re = fmaf(x.re, m.x, fmaf(x.im, m.y, r.re));
  r.im = fmaf(x.re, m.z, fmaf(x.im, m.w, r.im));
}
// sum_j conj(y_j) M1 + conj(M2) y_j from m = (M1r + M2r, M1i + M2i, M1i - M2i, M2r - M1r)
__device__ __forceinline__ void acc_col(cf& r, cf y, f4a m) { acc_row(r, y, m); }
// the 16 channels of knot row idx of sample b
template <bool BF16> __device__ __forceinline__ void load_knot(const DiagArgs& a, int b, int idx, float* x) {
  if constexpr (!BF16) {
    const f4a* r = reinterpret_cast<const f4a*>(reinterpret_cast<const float*>(a.path) + ((size_t)b * a.L + idx) * DIM);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const f4a v = r[i];
      x[4 * i] = v.x;
      x[4 * i + 1] = v.y;
      x[4 * i + 2] = v.z;
      x[4 * i + 3] = v.w;
    }
  } else {
    const f4a* r = reinterpret_cast<const f4a*>(reinterpret_cast<const unsigned short*>(a.path) +
                                                ((size_t)b * a.L + idx) * DIM);
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const f4a w = r[i];
      const float e[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        x[8 * i + 2 * q] = bf_lo(e[q]);
        x[8 * i + 2 * q + 1] = bf_hi(e[q]);
      }
    }
  }
}

// wave-wide scans on DPP: row shifts inside rows of 16 lanes, then the row broadcasts of lanes 15 and 31
template <int CTRL, int ROWS> __device__ __forceinline__ float dpp0(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROWS, 0xf, true));
}
__device__ __forceinline__ float wave_prefix(float v) {  // inclusive prefix sum over the 64 lanes
  v += dpp0<0x111, 0xf>(v);  // row_shr:1
  v += dpp0<0x112, 0xf>(v);  // row_shr:2
  v += dpp0<0x114, 0xf>(v);  // row_shr:4
  v += dpp0<0x118, 0xf>(v);  // row_shr:8
  v += dpp0<0x142, 0xa>(v);  // row_bcast:15 into rows 1 and 3
  v += dpp0<0x143, 0xc>(v);  // row_bcast:31 into rows 2 and 3
  return v;
}
__device__ __forceinline__ float lane63(float v) { return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63)); }
__device__ __forceinline__ float from_prev_lane(float v) { return dpp0<0x138, 0xf>(v); }  // wave_shr:1, lane 0 gets 0

typedef float f4m __attribute__((ext_vector_type(4)));
__device__ __forceinline__ f4m mfma4(float a, float b, f4m c) { return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0); }
// out (64 x 16) = in (64 x 16) M^T for a real 16 x 16 matrix given as its B-operand registers bm[ks] (lane l: M[l % 16]
// [4 ks + l / 16]): four row tiles of 16 steps, four 16x16x4 MFMAs each; the result goes to LDS, row-major.
// The per-step arrays are 64 rows of 16 floats without padding (three of them and the rest of the kernel's LDS stay
// under the 13 KB that lets three workgroups share a SIMD); entry (t, c) sits at column swz(t, c), an XOR of the
// column with an even value taken from t, so that 16 consecutive rows read at one column hit 16 distinct bank pairs
// and the complex pairs (2 j, 2 j + 1) stay adjacent.
constexpr int SP = DIM;
__device__ __forceinline__ int swz(int t, int c) { return c ^ (2 * ((t >> 1) & 7)); }
__device__ __forceinline__ void mfma_rows(const float (*in)[SP], const float* bm, float (*out)[SP], int l) {
  const int li = l & 15, lk = l >> 4;
#pragma unroll
  for (int tt = 0; tt < 4; ++tt) {
    f4m acc = {0.0f, 0.0f, 0.0f, 0.0f};
    const int ti = 16 * tt + li;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) acc = mfma4(in[ti][swz(ti, 4 * ks + lk)], bm[ks], acc);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int to = 16 * tt + 4 * lk + r;
      out[to][swz(to, li)] = acc[r];
    }
  }
}

// the same with in = sigma = (phi_k / 2) pi_k formed while loading the operand (phk: s_pl[.][2])
__device__ __forceinline__ void mfma_rows_sigma(const float (*pi)[SP], const float2 (*pl)[6], const float* bm,
                                                float (*out)[SP], int l) {
  const int li = l & 15, lk = l >> 4;
#pragma unroll
  for (int tt = 0; tt < 4; ++tt) {
    f4m acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      const int q = 4 * ks + lk, kq = q >> 1, ti = 16 * tt + li;
      const float2 x = *reinterpret_cast<const float2*>(&pi[ti][swz(ti, 2 * kq)]);
      const float2 hk = pl[kq][2];
      const float sv = (q & 1) ? fmaf(hk.x, x.y, hk.y * x.x) : fmaf(hk.x, x.x, -hk.y * x.y);
      acc = mfma4(sv, bm[ks], acc);
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int to = 16 * tt + 4 * lk + r;
      out[to][swz(to, li)] = acc[r];
    }
  }
}

// e^x by the hardware exponential, sine and cosine while |Im x| <= 16 (their absolute error stays near 1e-6 of
// |e^x| there), else the accurate library path
__device__ __forceinline__ cf expv_fast(cf x) {
  if (fabsf(x.im) > 16.0f) return expv(x);
  const float m = __expf(x.re);
  return cf{m * __cosf(x.im), m * __sinf(x.im)};
}

template <bool BF16>
__global__ __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(3))) void k_bwd_carry(DiagArgs a) {
  // per step: pi, gamma; then s_o: the matrices, then each MFMA result in turn (rows swizzled by swz)
  __shared__ __align__(16) float s_buf[3][kMaxT][SP];
  float(*s_pi)[SP] = s_buf[0];
  float(*s_ga)[SP] = s_buf[1];
  float(*s_o)[SP] = s_buf[2];
  __shared__ __align__(16) float2 s_wh[kMaxT];
  __shared__ __align__(16) float2 s_pl[K][6];  // per plane: rho, phi, phi/2, lam1, e^{u tau} C1, 1/rho
  f4a(*s_mat)[K][K] = reinterpret_cast<f4a(*)[K][K]>(&s_o[0][0]);  // s_mr, s_gr, s_mc, s_gc: 4 KB
  const int l = threadIdx.x, c = blockIdx.x, b = blockIdx.y;
  const int jj = l >> 3, kk = l & 7;
  const int flag = a.cflag[b * a.C + c];
  const bool owned = (flag & 3) == 3;  // a pair-group chunk with invertible steps (else the generic kernels)
  const int t0 = c * a.T, Tc = min(a.T, a.n_int - t0);
  const float* th = a.clock + (size_t)b * a.L + t0;
  // ---- lane = step t: this step's inputs and local dv, loaded before the carry chain below
  const int t = l;
  const bool live = owned && t < Tc;
  float h = 0.0f, hs = 0.0f, th_end = 0.0f, tau = 0.0f;
  float x0[DIM], x1[DIM];
#pragma unroll
  for (int i = 0; i < DIM; ++i) x0[i] = x1[i] = 0.0f;
  if (owned) {
    th_end = th[Tc];
    tau = th_end - th[0];
  }
  if (live) {
    h = th[t + 1] - th[t];
    hs = th_end - th[t + 1];
    load_knot<BF16>(a, b, t0 + t, x0);
    load_knot<BF16>(a, b, t0 + t + 1, x1);
  }
  // adjoint carry inside the quad (float64, lane = 8 j + k): the cotangent on this chunk's end state, down from the
  // quad's last chunk (written by the adjoint scan); written back for every later kernel that reads mt
  // (every operand of the up to three steps is loaded before the first one: the loads do not depend on the chain)
  const int c_last = min(4 * (c / 4) + 3, a.C - 1), nstep = c_last - c;
  PairSt X = load_st_f(a.mt + ((size_t)b * a.C + c_last) * a.D, jj, kk);
  dc sFj[3], sFk[3], sC0[3], sC1[3];
  PairSt sMu[3];
#pragma unroll
  for (int i = 0; i < 3; ++i) {
    if (i < nstep) {
      const int cc = c_last - 1 - i;
      const double* cfl = a.cflow + ((size_t)b * a.C + cc + 1) * K * 2;
      sFj[i] = ld_dd(cfl + 2 * jj);
      sFk[i] = ld_dd(cfl + 2 * kk);
      sC0[i] = ld_dd(a.carries + ((size_t)b * (a.C + 1) + cc + 1) * a.D + 2 * kk);
      sC1[i] = ld_dd(a.carries + ((size_t)b * (a.C + 1) + cc + 2) * a.D + 2 * kk);
      sMu[i] = load_st_f(a.mu + ((size_t)b * a.C + cc + 1) * a.D, jj, kk);
    }
  }
#pragma unroll
  for (int i = 0; i < 3; ++i) {
    if (i < nstep) {  // uniform over the wave: the shuffles inside adj_d see every lane
      adj_d(X, sFj[i], sFk[i], sC1[i] - sFk[i] * sC0[i]);  // level-1 increment carry1(cc+2) - F carry1(cc+1)
      add_st(X, sMu[i]);
    }
  }
  if (c < c_last) store_st_f(a.mt + ((size_t)b * a.C + c) * a.D, jj, kk, X);
  if (!owned) return;
  const PairCoefs pc = pair_coefs(a, jj, kk, a.chbar[b * a.C + c], (flag & 4) != 0);
  const double* cr0 = a.carries + ((size_t)b * (a.C + 1) + c) * a.D;  // carry-in state
  const cf lB{(float)(2.0 * X.SB.re), (float)(2.0 * X.SB.im)}, lA{(float)(2.0 * X.SA.re), (float)(2.0 * X.SA.im)};
  {
    const cf GB = cjm(pc.IB, lB), GA = cjm(pc.IA, lA);
    s_mat[0][jj][kk] = f4a{lB.re + lA.re, lB.im - lA.im, lB.im + lA.im, lA.re - lB.re};
    s_mat[1][jj][kk] = f4a{GB.re + GA.re, GB.im - GA.im, GB.im + GA.im, GA.re - GB.re};
    s_mat[2][jj][kk] = f4a{lB.re + lA.re, lB.im + lA.im, lB.im - lA.im, lA.re - lB.re};
    s_mat[3][jj][kk] = f4a{GB.re + GA.re, GB.im + GA.im, GB.im - GA.im, GA.re - GB.re};
    if (kk == 0) {
      const cf E = expv(tau * load_u(a.params, jj)) * cf{(float)cr0[2 * jj], (float)cr0[2 * jj + 1]};
      const cf ri = cf{1.0f, 0.0f} / pc.rho_j;
      s_pl[jj][0] = float2{pc.rho_j.re, pc.rho_j.im};
      s_pl[jj][1] = float2{pc.phi_j.re, pc.phi_j.im};
      s_pl[jj][3] = float2{(float)X.S1.re, (float)X.S1.im};
      s_pl[jj][4] = float2{E.re, E.im};
      s_pl[jj][5] = float2{ri.re, ri.im};
    }
    if (jj == 0) s_pl[kk][2] = float2{pc.phk_k.re, pc.phk_k.im};
  }
  cf pi[K], fl[K];  // fl = e^{u n_t} = conj(a_t): plane flows over the clock span after step t
#pragma unroll
  for (int j = 0; j < K; ++j) {
    // pi = p conj(a): p times the plane flow over the clock span after step t
    fl[j] = live ? expv_fast(hs * load_u(a.params, j)) : cf{0.0f, 0.0f};
    pi[j] = cf{x1[2 * j] - x0[2 * j], x1[2 * j + 1] - x0[2 * j + 1]} * fl[j];
  }
  __syncthreads();
  // B operands of the matvec products: lane l holds M[p][q], p = l % 16, q = 4 ks + l / 16. Rows: out_j = sum_k
  // block(j,k) in_k with block(j,k)[a][b] the (a, b) entry of s_mat[0 | 1][j][k]; columns: out_k = sum_j
  // block(j,k) in_j with s_mat[2 | 3][j][k].
  float bmr[4], bgr[4], bmc[4], bgc[4];
  {
    const int pp = l & 15;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      const int q = 4 * ks + (l >> 4), e = 2 * (pp & 1) + (q & 1);
      bmr[ks] = reinterpret_cast<const float*>(&s_mat[0][pp >> 1][q >> 1])[e];
      bgr[ks] = reinterpret_cast<const float*>(&s_mat[1][pp >> 1][q >> 1])[e];
      bmc[ks] = reinterpret_cast<const float*>(&s_mat[2][q >> 1][pp >> 1])[e];
      bgc[ks] = reinterpret_cast<const float*>(&s_mat[3][q >> 1][pp >> 1])[e];
    }
  }
  // gamma_t = c_t conj(a_t) = e^{u tau} C1 + phi sum_{s<t} pi_s (the flows telescope)
  cf ga[K];
#pragma unroll
  for (int j = 0; j < K; ++j) {
    const float2 f = s_pl[j][1], e = s_pl[j][4];
    const cf ex{wave_prefix(pi[j].re) - pi[j].re, wave_prefix(pi[j].im) - pi[j].im};
    ga[j] = live ? fma_c(cf{f.x, f.y}, ex, cf{e.x, e.y}) : cf{0.0f, 0.0f};
    *reinterpret_cast<float2*>(&s_pi[t][swz(t, 2 * j)]) = float2{pi[j].re, pi[j].im};
    *reinterpret_cast<float2*>(&s_ga[t][swz(t, 2 * j)]) = float2{ga[j].re, ga[j].im};
  }
  s_wh[t] = float2{h, hs};
  __syncthreads();  // the matrices are in registers; s_o is free
  // rows: RC_t = M_R sigma_t (level-1 cotangent terms), RP_t = G_R pi_t (plane part of dv)
  float rc[DIM], rp[DIM];
  mfma_rows_sigma(s_pi, s_pl, bmr, s_o, l);
  __syncthreads();
#pragma unroll
  for (int i = 0; i < DIM; ++i) rc[i] = s_o[t][swz(t, i)];
  __syncthreads();
  mfma_rows(s_pi, bgr, s_o, l);
  __syncthreads();
#pragma unroll
  for (int i = 0; i < DIM; ++i) rp[i] = s_o[t][swz(t, i)];
  __syncthreads();
  // columns: the later factor's part of dv, CA_t = M_C gamma_t, CB_t = G_C pi_t (CA waits in s_o, CB in registers)
  mfma_rows(s_ga, bmc, s_o, l);
  float dvt[DIM];
  cf kphj_p{0.0f, 0.0f}, krho_p{0.0f, 0.0f};  // plane kk's sums (lanes kk < K use them)
#pragma unroll
  for (int j = 0; j < K; ++j) {
    const cf RC{rc[2 * j], rc[2 * j + 1]}, RP{rp[2 * j], rp[2 * j + 1]};
    // sums of RC over the steps after t (excl) and from t on (incl): the total minus the inclusive prefix
    const float pr = wave_prefix(RC.re), pim = wave_prefix(RC.im);
    const cf excl{lane63(pr) - pr, lane63(pim) - pim};
    const cf incl = excl + RC;
    const float2 f = s_pl[j][1], l1e = s_pl[j][3], ri = s_pl[j][5];
    const cf lam1{l1e.x, l1e.y};
    const cf ex = lam1 + excl;
    const cf dvp = conj(fl[j]) * fma_c(conj(cf{f.x, f.y}), ex, RP);
    dvt[2 * j] = dvp.re;
    dvt[2 * j + 1] = dvp.im;
    // kphj += h conj(pi) (lam1 + excl); krho += h conj(S1(t-1)) a (lam1 + incl), S1(t-1) conj(a) = gamma / rho
    const cf q1 = h * cjm(pi[j], ex);
    const cf q2 = h * cjm(ga[j] * cf{ri.x, ri.y}, lam1 + incl);
    const cf s1{lane63(wave_prefix(q1.re)), lane63(wave_prefix(q1.im))};
    const cf s2{lane63(wave_prefix(q2.re)), lane63(wave_prefix(q2.im))};
    if (j == kk) {
      kphj_p = s1;
      krho_p = s2;
    }
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < DIM; ++i) rc[i] = s_o[t][swz(t, i)];  // CA
  __syncthreads();
  // the step's local dv (written by the local adjoint), loaded here rather than with the inputs to keep the
  // registers of the steps above free; this lane overwrites the same row with the total below
  float dvl[DIM];
  {
    const f4a* dvr = reinterpret_cast<const f4a*>(a.dv + ((size_t)b * a.n_int + t0 + (live ? t : 0)) * DIM);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const f4a v = live ? dvr[i] : f4a{0.0f, 0.0f, 0.0f, 0.0f};
      dvl[4 * i] = v.x;
      dvl[4 * i + 1] = v.y;
      dvl[4 * i + 2] = v.z;
      dvl[4 * i + 3] = v.w;
    }
  }
  mfma_rows(s_pi, bgc, s_o, l);
  __syncthreads();
#pragma unroll
  for (int k = 0; k < K; ++k) {
    const float2 hk = s_pl[k][2];
    const cf col = conj(fl[k]) * fma_c(conj(cf{hk.x, hk.y}), cf{rc[2 * k], rc[2 * k + 1]},
                                       cf{s_o[t][swz(t, 2 * k)], s_o[t][swz(t, 2 * k + 1)]});
    dvt[2 * k] += col.re + dvl[2 * k];
    dvt[2 * k + 1] += col.im + dvl[2 * k + 1];
  }
  if (live) {
    float* dvr = a.dv + ((size_t)b * a.n_int + t0 + t) * DIM;
#pragma unroll
    for (int i = 0; i < DIM; i += 4) *reinterpret_cast<f4a*>(dvr + i) = f4a{dvt[i], dvt[i + 1], dvt[i + 2], dvt[i + 3]};
  }
  // interior knots t0 + 1 .. t0 + Tc - 1: dX_t = dv(t-1) - dv(t); the boundary knots are finished by k_knot_grads
  {
    float dk[DIM];
#pragma unroll
    for (int i = 0; i < DIM; ++i) dk[i] = from_prev_lane(dvt[i]) - dvt[i];
    if (live && t >= 1) {
      float* kr = a.dpath + ((size_t)b * a.L + t0 + t) * DIM;
#pragma unroll
      for (int i = 0; i < DIM; i += 4) *reinterpret_cast<f4a*>(kr + i) = f4a{dk[i], dk[i + 1], dk[i + 2], dk[i + 3]};
    }
  }
  __syncthreads();
  // ---- outer-product sums over the steps on MFMA: D[m][n] = sum_t x_t[m] (w_t pi_t[n]) for x = pi, gamma and
  // w = h, n (16 x 16 real, all four real products of each complex pair), sixteen k-steps of four steps each
  {
    const int li = l & 15, lk = l >> 4;
    f4m d1 = {0.0f, 0.0f, 0.0f, 0.0f}, d2 = d1, d3 = d1, d4 = d1;
#pragma unroll 4
    for (int ks = 0; ks < kMaxT / 4; ++ks) {
      const int ts = 4 * ks + lk;
      const float xp = s_pi[ts][swz(ts, li)], xg = s_ga[ts][swz(ts, li)];
      const float2 w = s_wh[ts];
      const float yh = w.x * xp, ys = w.y * xp;
      d1 = mfma4(xp, yh, d1);
      d2 = mfma4(xp, ys, d2);
      d3 = mfma4(xg, yh, d3);
      d4 = mfma4(xg, ys, d4);
    }
    __syncthreads();  // gamma and the MFMA results are no longer read
    float(*dd)[16][17] = reinterpret_cast<float(*)[16][17]>(&s_buf[1][0][0]);  // 4 x 16 x 17 <= 2 x 64 x SP
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      dd[0][4 * lk + r][li] = d1[r];
      dd[1][4 * lk + r][li] = d2[r];
      dd[2][4 * lk + r][li] = d3[r];
      dd[3][4 * lk + r][li] = d4[r];
    }
  }
  __syncthreads();
  // ---- lane = pair (jj, kk)
  const float(*dd)[16][17] = reinterpret_cast<const float(*)[16][17]>(&s_buf[1][0][0]);
  // x y = (rr - ii, ri + ir), x conj(y) = (rr + ii, ir - ri), with rr = D[2j][2k], ii = D[2j+1][2k+1], ...
  cf P[4], Pc[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const float rr = dd[q][2 * jj][2 * kk], ii = dd[q][2 * jj + 1][2 * kk + 1];
    const float ri = dd[q][2 * jj][2 * kk + 1], ir = dd[q][2 * jj + 1][2 * kk];
    P[q] = cf{rr - ii, ri + ir};
    Pc[q] = cf{rr + ii, ir - ri};
  }
  // P[0] = sum h pi_j pi_k, P[1] = sum n pi_j pi_k, P[2] = sum h gamma_j pi_k, P[3] = sum n gamma_j pi_k
  const cf kIB = lB * conj(P[0]), kIA = lA * conj(Pc[0]);
  const cf kph = lB * conj(P[2]) + conj(lA) * Pc[2];
  const double* cr = cr0 + DIM + 4 * (8 * jj + kk);
  const cf C2Ah{(float)(0.5 * cr[0]), (float)(0.5 * cr[1])}, C2Bh{(float)(0.5 * cr[2]), (float)(0.5 * cr[3])};
  const cf uj = load_u(a.params, jj), uk = load_u(a.params, kk);
  const cf WB = (tau * (C2Bh * expv(tau * (uj + uk))) + pc.phk_k * P[3] + pc.IB * P[1]) / pc.LB;
  const cf WA = (tau * (C2Ah * expv(tau * (uj + conj(uk)))) + conj(pc.phk_k) * Pc[3] + pc.IA * Pc[1]) / pc.LA;
  const cf kLB = lB * conj(WB), kLA = lA * conj(WA);
  // coefficient cotangents -> parameter partials (d_j, w_j), as k_bwd_full: a node h u contributes (-Re G, Im G)
  // for u = -conj(z) and (-Re G, -Im G) for u = -z (the conj(u_k) of the A pairs)
  const cf Gx = 0.5f * (kIB * conj(pc.DxB) + kIA * conj(pc.DxA));
  const cf GyB = 0.5f * (kIB * conj(pc.DyB)) + kLB * conj(pc.LB);
  const cf GyA = 0.5f * (kIA * conj(pc.DyA)) + kLA * conj(pc.LA);
  const cf Gk = 0.5f * (kph * conj(pc.dphi_k));
  f4a* s_part = reinterpret_cast<f4a*>(&s_pi[0][0]);  // pi is no longer read
  s_part[l] = f4a{-GyB.re - GyA.re - Gx.re, GyB.im + GyA.im + Gx.im, -GyB.re - GyA.re - Gk.re, GyB.im - GyA.im + Gk.im};
  __syncthreads();
  if (l < K) {
    const int pl = l;  // plane: rows (pl, k) and columns (j, pl)
    float sd = 0.0f, sw = 0.0f;
    for (int q = 0; q < K; ++q) {
      const f4a r = s_part[8 * pl + q], cl = s_part[8 * q + pl];
      sd += r.x + cl.z;
      sw += r.y + cl.w;
    }
    const float2 r = s_pl[pl][0];
    const cf Gp = krho_p * conj(cf{r.x, r.y}) + kphj_p * conj(pc.dphi_k);  // lane pl: jj = 0, kk = pl
    sd -= Gp.re;
    sw += Gp.im;
    float* gpo = a.gp + ((size_t)b * a.C + c) * a.npar;
    gpo[2 * pl] += sd;
    gpo[2 * pl + 1] += sw;
  }
}

// ------------------------------------------------------------------------------------------------ look-back forward
// The whole forward in one launch: one workgroup (one wavefront) per quad of four chunks; its sample comes from
// the workgroup index and its quad from the sample's ticket counter, so that a quad waits only on quads whose
// workgroups already run (per-sample counters on separate cache lines keep the tickets from serialising):
//   A. every chunk's classification and its summary from a zero state;
//   B. the quad's aggregate in float64 (lane = 8 j + k), published (status 1);
//   C. the look-back: the quad's carry is the fold of the aggregates of the earlier quads of its group of LBG quads
//      and of the aggregates of the earlier groups; the last quad of a group publishes its group's aggregate (the
//      fold of the group's quads) on the way. At most LBG - 1 + (quads / LBG) folds per quad, and no quad waits on
//      another's look-back but for the group aggregates, each LBG - 1 folds after its quads' own aggregates;
//   D. the chunk carries inside the quad (written for the backward) and the prefix rows.
// The chunk summaries of some quads overlap other quads' row writes, and the carry scans between passes disappear.
// Publication: every aggregate word starts as the sentinel kLbEmpty (k_coef_table fills the buffer; it runs first in
// the same stream) and is written once per call by an agent-scope relaxed atomic store (coherent across the XCDs'
// L2s with no cache write-back); readers load each word with an agent-scope atomic load and take it only when it is
// not the sentinel, re-reading until it is. Correctness rests on each word alone (one store per location, after the
// fill), not on an ordering between locations, so no release/acquire pair is needed (a release at agent scope
// writes back the XCD's dirty L2 lines: +75 us on this kernel, whose rows fill the L2). The status word is only the
// hint of when to start reading: it is set after a wait on the wavefront's outstanding stores, so the reads
// normally find every word already there. The status words and the ticket are zeroed by k_coef_table. Uniform
// quads run the 16-lane groups (KP = 4, coefficients at each chunk's mean step); a quad with a non-uniform chunk
// runs one lane per pair (lane = 8 j + k) with every step's coefficients at its own clock step, chunk by chunk.

__device__ __forceinline__ bool lb_empty(double v) { return (unsigned long long)__double_as_longlong(v) == kLbEmpty; }
__device__ __forceinline__ bool lb_empty(dc v) { return lb_empty(v.re) | lb_empty(v.im); }
__device__ __forceinline__ void pub_d(double* p, dc v) {
  __hip_atomic_store(p, v.re, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __hip_atomic_store(p + 1, v.im, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ dc sub_d(const double* p) {
  return dc{__hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT),
            __hip_atomic_load(p + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)};
}
__device__ __forceinline__ void pub_st(double* row, int j, int k, const PairSt& s) {
  if (k == 0) pub_d(row + 2 * j, s.S1);
  pub_d(row + poff(j, k), s.SA);
  pub_d(row + poff(j, k) + 2, s.SB);
}
__device__ __forceinline__ PairSt sub_st(const double* row, int j, int k) {
  return PairSt{sub_d(row + 2 * j), sub_d(row + poff(j, k)), sub_d(row + poff(j, k) + 2)};
}
// an aggregate (state, then its K plane flows from offset D) with status word w
__device__ __forceinline__ void publish(double* row, int* w, int D, int j, int k, const PairSt& s, dc Fj) {
  pub_st(row, j, k, s);
  if (k == 0) pub_d(row + D + 2 * j, Fj);
  __builtin_amdgcn_s_waitcnt(0);  // the wavefront's published words have landed (the status is a hint only)
  if (threadIdx.x == 0) __hip_atomic_store(w, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ dc shfl_d(dc v, int src) { return dc{__shfl(v.re, src), __shfl(v.im, src)}; }

// a wait that reached kSpinLimit sets the coefficient table's error word (read by ews_diag_forward_status)
__device__ __forceinline__ void lb_timeout(const DiagArgs& a) {
  if (threadIdx.x == 0)
    __hip_atomic_store(reinterpret_cast<int*>(a.ctab) + kCtabStatus, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// The look-back items of quad q, latest first: items 0 .. nq-1 the earlier quads of its group (q-1 down to its
// group's first quad), then items nq .. nq+ng-1 the earlier groups (g-1 down to 0).
struct LbItems {
  const double* qrow;  // quad aggregates of the sample
  const double* grow;  // group aggregates of the sample
  const int* qst;      // their status words
  const int* gst;
  int q, g, nq, ng;
  size_t AW;
};
__device__ __forceinline__ const double* item_row(const LbItems& it, int i) {
  return i < it.nq ? it.qrow + (size_t)(it.q - 1 - i) * it.AW : it.grow + (size_t)(it.g - 1 - (i - it.nq)) * it.AW;
}
__device__ __forceinline__ const int* item_status(const LbItems& it, int i) {
  return i < it.nq ? it.qst + (it.q - 1 - i) : it.gst + (it.g - 1 - (i - it.nq));
}
// acc <- (items i0 .. i1-1 folded, latest first) (x) acc, with the flows of the folded span in aFj, aFk; the items'
// status words have been seen nonzero. A batch is re-read while any of its words is still the sentinel; false if that
// lasts kSpinLimit reads.
__device__ __forceinline__ bool lb_fold(const LbItems& it, int i0, int i1, int D, int j, int k, PairSt& acc, dc& aFj,
                                        dc& aFk) {
  for (int b0 = i0; b0 < i1; b0 += LBB) {
    PairSt g[LBB];
    dc gFj[LBB], gFk[LBB];
    for (int polls = 0;; ++polls) {
      bool empty = false;
#pragma unroll
      for (int u = 0; u < LBB; ++u) {
        if (b0 + u < i1) {
          const double* gr = item_row(it, b0 + u);
          g[u] = sub_st(gr, j, k);
          gFj[u] = sub_d(gr + D + 2 * j);
          gFk[u] = sub_d(gr + D + 2 * k);
          empty |= lb_empty(g[u].S1) | lb_empty(g[u].SA) | lb_empty(g[u].SB) | lb_empty(gFj[u]) | lb_empty(gFk[u]);
        }
      }
      if (!__any(empty)) break;
      if (polls >= kSpinLimit) return false;
      __builtin_amdgcn_s_sleep(1);
    }
#pragma unroll
    for (int u = 0; u < LBB; ++u) {
      if (b0 + u < i1) {  // the item (earlier) followed by the folded span (later)
        chen_d(g[u], aFj, aFk, acc.S1, shfl_d(acc.S1, 8 * k), acc.SA, acc.SB);
        acc = g[u];
        aFj = gFj[u] * aFj;
        aFk = gFk[u] * aFk;
      }
    }
  }
  return true;
}
// fold items [i0, i1) as their status words turn nonzero: one load per lane reads up to 64 of them at once
__device__ __forceinline__ bool lb_fold_ready(const LbItems& it, int i0, int i1, int D, int j, int k, PairSt& acc,
                                             dc& aFj, dc& aFk) {
  int polls = 0;
  while (i0 < i1) {
    const int i = i0 + (int)threadIdx.x;
    const int sv = i < i1 ? __hip_atomic_load(item_status(it, i), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 1;
    const unsigned long long notready = __ballot(sv == 0);
    const int nr = notready ? __ffsll((long long)notready) - 1 : 64;  // leading items already published
    const int n = min(nr, i1 - i0);
    if (!lb_fold(it, i0, i0 + n, D, j, k, acc, aFj, aFk)) return false;
    i0 += n;
    if (n == 0) {
      if (++polls >= kSpinLimit) return false;
      __builtin_amdgcn_s_sleep(1);
    }
  }
  return true;
}

// The steps of the group's chunk from the lane states (S1; halved pair states SA, SB) at the chunk's mean-step
// coefficients: the summary recursion (OUT false) or the prefix rows (OUT true, row staging in buf). The staged
// increments are shared by the wavefront: every lane runs every block, and a group whose chunk is absent only skips
// the arithmetic.
template <bool OUT, bool BF16>
__device__ __forceinline__ void lb_steps(const DiagArgs& a, const Lane& l, int b, int cb, int t0, int Tc,
                                         const FwdCoef<4>& f, cf& S1, cf* SA, cf* SB_, float (*s_v)[4 * VBLK],
                                         float* buf) {
  constexpr int KP = 4, GPW = 4;
  VRaw<GPW, BF16> vr;
  vblk_load<GPW, BF16>(a, b, cb, 0, vr);
  vblk_store<GPW, BF16>(a, cb, 0, vr, s_v[0]);
  wave_order();
  float* orow = a.out + ((size_t)b * a.n_int + t0) * a.W;
  const int o1 = a.off1 + 2 * l.j;
  const int nblk = (a.T + SB - 1) / SB;
  for (int blk = 0; blk < nblk; ++blk) {
    if (blk + 1 < nblk) vblk_load<GPW, BF16>(a, b, cb, blk + 1, vr);
    const float* vg = s_v[blk & 1] + l.gi * VBLK;
    for (int st = 0; st < SB; ++st) {
      const int t = blk * SB + st;
      if (t >= Tc) break;
      cf pj, pk[KP];
      load_p<KP>(vg + st * DIM, l, pj, pk);
      const cf cj = f.rho * S1;
      S1 = fma_c(f.phi, pj, cj);
      static_for<0, KP>([&](auto qc) {
        constexpr int q = qc;
        const cf sg = f.phk[q] * pk[q];
        cf pi, pic;
        prods(pj, pk[q], pi, pic);
        SB_[q] = fma_c(f.LB[q], SB_[q], fma_c(cj, sg, f.IB[q] * pi));
        SA[q] = fma_c(f.LA[q], SA[q], fma_c(cj, conj(sg), f.IA[q] * pic));
      });
      if constexpr (OUT) {
        float* row = orow + (size_t)t * a.W;
        if (a.lvl0 && l.gl == 0) row[0] = 1.0f;
        if (l.kg == 0) *reinterpret_cast<f2u*>(row + o1) = f2u{S1.re, S1.im};
        f4a* p0 = reinterpret_cast<f4a*>(buf + row_at(2 * l.j) + 2 * KP * l.kg);
        f4a* p1 = reinterpret_cast<f4a*>(buf + row_at(2 * l.j + 1) + 2 * KP * l.kg);
        static_for<0, KP / 2>([&](auto ic) {
          constexpr int i = ic, q0 = 2 * i, q1 = 2 * i + 1;
          p0[i] = f4a{SA[q0].re + SB_[q0].re, SB_[q0].im - SA[q0].im, SA[q1].re + SB_[q1].re, SB_[q1].im - SA[q1].im};
          p1[i] = f4a{SA[q0].im + SB_[q0].im, SA[q0].re - SB_[q0].re, SA[q1].im + SB_[q1].im, SA[q1].re - SB_[q1].re};
        });
        wave_order();
        float* row2 = row + a.off2;
        static_for<0, Pieces<KP>::NP>([&](auto ic) {
          constexpr int i = ic;
          const int pi = l.gl + Geo<KP>::G * i;
          const f4a v = *reinterpret_cast<const f4a*>(buf + piece_at(pi));
          *reinterpret_cast<f4u*>(row2 + 4 * pi) = f4u{v.x, v.y, v.z, v.w};
        });
        wave_order();
      }
    }
    if (blk + 1 < nblk) vblk_store<GPW, BF16>(a, cb, blk + 1, vr, s_v[(blk + 1) & 1]);
    wave_order();
  }
}

// The summary of a uniform chunk from a zero state in closed form, lane t = step t of the chunk. With the span
// n_t = theta_end - theta_{t+1} after step t, pi_t = p_t e^{u n_t} (per plane) and its exclusive prefix sum
// P_t = sum_{s<t} pi_s over the steps (the flows telescope: e^{u n_t} c_t = phi P_t for the level-1 state
// c_t = rho S1(t-1) before step t), the chunk's full-scale summary is
//   S1_j = phi_j sum_t pi_{t,j},
//   SB_jk = phi_j phi_k sum_t P_{t,j} pi_{t,k} + IB_jk sum_t pi_{t,j} pi_{t,k},
//   SA_jk = phi_j conj(phi_k) sum_t P_{t,j} conj(pi_{t,k}) + IA_jk sum_t pi_{t,j} conj(pi_{t,k}),
// with the coefficients at the chunk's mean step. The two sums over t are real 16 x 16 outer-product sums on fp32
// MFMA (every complex product is a combination of their four real products). Writes the summary in the layout of
// s_row (level 1 at 2 j, pair (j, k) at poff).
// The lane's operands of one chunk's closed form (lane t = step t): its knots and the clock span after the step.
template <bool BF16> struct CfIn {
  float x0[DIM], x1[DIM], n;
};
template <bool BF16>
__device__ __forceinline__ void lb_cf_load(const DiagArgs& a, int b, int c, CfIn<BF16>& in) {
  const int l = threadIdx.x, t0 = c * a.T, Tc = min(a.T, a.n_int - t0);
  const float* th = a.clock + (size_t)b * a.L + t0;
  if (l < Tc) {
    load_knot<BF16>(a, b, t0 + l, in.x0);
    load_knot<BF16>(a, b, t0 + l + 1, in.x1);
    in.n = th[Tc] - th[l + 1];
  }
}
// the lane's (lane = 8 j + k) coefficients of the closed form from the coefficient table (read once per quad)
struct CfTab {
  cf phj, phk, IB, IA;
};
__device__ __forceinline__ CfTab cf_tab(const DiagArgs& a, int j, int k) {
  return CfTab{tp(a.ctab, j, TP_PHI), tp(a.ctab, k, TP_PHI), 2.0f * tq(a.ctab, j, k, TQ_IB),
               2.0f * tq(a.ctab, j, k, TQ_IA)};
}
template <bool BF16>
__device__ __forceinline__ void lb_summary_cf(const DiagArgs& a, int b, int c, float hb, bool use_tab,
                                              const CfTab& ct, const CfIn<BF16>& in, float (*s_x)[DIM],
                                              float (*s_y)[DIM], float* s_tot, float* sp) {
  const int l = threadIdx.x, t0 = c * a.T, Tc = min(a.T, a.n_int - t0);
  float pv[DIM];
#pragma unroll
  for (int i = 0; i < DIM; ++i) pv[i] = 0.0f;
  if (l < Tc) {
#pragma unroll
    for (int j = 0; j < K; ++j) {
      const cf v =
          cf{in.x1[2 * j] - in.x0[2 * j], in.x1[2 * j + 1] - in.x0[2 * j + 1]} * expv_fast(in.n * load_u(a.params, j));
      pv[2 * j] = v.re;
      pv[2 * j + 1] = v.im;
    }
  }
#pragma unroll
  for (int i = 0; i < DIM; ++i) {
    const float inc = wave_prefix(pv[i]);
    s_y[l][i] = pv[i];
    s_x[l][i] = inc - pv[i];
    if (l == Tc - 1) s_tot[i] = inc;
  }
  __syncthreads();
  // dd[0] = sum_t P_t (x) pi_t, dd[1] = sum_t pi_t (x) pi_t: sixteen k-steps of four steps each; the results
  // overwrite the start of s_x once every operand has been read (one wavefront: LDS operations in program order)
  float(*s_dd)[16][17] = reinterpret_cast<float(*)[16][17]>(&s_x[0][0]);
  {
    const int li = l & 15, lk = l >> 4;
    f4m d1 = {0.0f, 0.0f, 0.0f, 0.0f}, d2 = d1;
#pragma unroll 4
    for (int ks = 0; ks < kMaxT / 4; ++ks) {
      const int ts = 4 * ks + lk;
      const float xv = s_x[ts][li], yv = s_y[ts][li];
      d1 = mfma4(xv, yv, d1);
      d2 = mfma4(yv, yv, d2);
    }
    wave_order();
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      s_dd[0][4 * lk + r][li] = d1[r];
      s_dd[1][4 * lk + r][li] = d2[r];
    }
  }
  __syncthreads();
  const int j = l >> 3, k = l & 7;
  cf phj, phk, IB, IA;
  if (use_tab) {
    phj = ct.phj;
    phk = ct.phk;
    IB = ct.IB;
    IA = ct.IA;
  } else {
    const cf uj = load_u(a.params, j), uk = load_u(a.params, k), xj = hb * uj;
    phj = node1(xj).p;
    phk = node1(hb * uk).p;
    IB = dd3<cf, false>(xj, hb * (uj + uk)).d;
    IA = dd3<cf, false>(xj, hb * (uj + conj(uk))).d;
  }
  cf X, Xc, Y, Yc;  // sum x_j y_k and sum x_j conj(y_k) of dd[0] (X) and dd[1] (Y)
  {
    const float rr = s_dd[0][2 * j][2 * k], ii = s_dd[0][2 * j + 1][2 * k + 1];
    const float ri = s_dd[0][2 * j][2 * k + 1], ir = s_dd[0][2 * j + 1][2 * k];
    X = cf{rr - ii, ri + ir};
    Xc = cf{rr + ii, ir - ri};
  }
  {
    const float rr = s_dd[1][2 * j][2 * k], ii = s_dd[1][2 * j + 1][2 * k + 1];
    const float ri = s_dd[1][2 * j][2 * k + 1], ir = s_dd[1][2 * j + 1][2 * k];
    Y = cf{rr - ii, ri + ir};
    Yc = cf{rr + ii, ir - ri};
  }
  const cf SBv = (phj * phk) * X + IB * Y;
  const cf SAv = (phj * conj(phk)) * Xc + IA * Yc;
  if (k == 0) {
    const cf S1 = phj * cf{s_tot[2 * j], s_tot[2 * j + 1]};
    *reinterpret_cast<float2*>(sp + 2 * j) = float2{S1.re, S1.im};
  }
  *reinterpret_cast<f4a*>(sp + poff(j, k)) = f4a{SAv.re, SAv.im, SBv.re, SBv.im};
  __syncthreads();  // the LDS scratch is reused by the next chunk
}

// A chunk of a quad that holds a non-uniform chunk, one lane per pair (lane = 8 j + k), every step's coefficients at
// its own clock step; the lane's full-scale states S1 (of plane j), SA, SB (of pair (j, k)) go in and out. OUT:
// the lane writes level 1 (k = 0) and its 2 x 2 block of every prefix row.
template <bool OUT, bool BF16>
__device__ __forceinline__ void lb_pairwise(const DiagArgs& a, int b, int c, int j, int k, dc& S1d, dc& SAd,
                                            dc& SBd) {
  const int t0 = c * a.T, Tc = min(a.T, a.n_int - t0);
  const float* th = a.clock + (size_t)b * a.L + t0;
  const cf uj = load_u(a.params, j), uk = load_u(a.params, k);
  const cf ub = uj + uk, ua = uj + conj(uk);
  cf S1{(float)S1d.re, (float)S1d.im}, SA{(float)SAd.re, (float)SAd.im}, SBv{(float)SBd.re, (float)SBd.im};
  for (int t = 0; t < Tc; ++t) {
    const size_t ix = (size_t)b * a.L + t0 + t;
    cf pj, pk;
    if constexpr (!BF16) {
      const float* x = reinterpret_cast<const float*>(a.path) + ix * DIM;
      pj = cf{x[DIM + 2 * j] - x[2 * j], x[DIM + 2 * j + 1] - x[2 * j + 1]};
      pk = cf{x[DIM + 2 * k] - x[2 * k], x[DIM + 2 * k + 1] - x[2 * k + 1]};
    } else {
      const unsigned short* x = reinterpret_cast<const unsigned short*>(a.path) + ix * DIM;
      auto bf = [](unsigned short v) { return __uint_as_float((unsigned)v << 16); };
      pj = cf{bf(x[DIM + 2 * j]) - bf(x[2 * j]), bf(x[DIM + 2 * j + 1]) - bf(x[2 * j + 1])};
      pk = cf{bf(x[DIM + 2 * k]) - bf(x[2 * k]), bf(x[DIM + 2 * k + 1]) - bf(x[2 * k + 1])};
    }
    const float h = th[t + 1] - th[t];
    const cf xj = h * uj;
    const Node1<cf> nj = node1(xj);
    const cf s1k = node1(h * uk).p * pk;
    const cf cj = nj.e * S1;
    SBv = expv(h * ub) * SBv + cj * s1k + dd3<cf, false>(xj, h * ub).d * (pj * pk);
    SA = expv(h * ua) * SA + cj * conj(s1k) + dd3<cf, false>(xj, h * ua).d * (pj * conj(pk));
    S1 = cj + nj.p * pj;
    if constexpr (OUT) {
      float* row = a.out + ((size_t)b * a.n_int + t0 + t) * a.W;
      if (a.lvl0 && j == 0 && k == 0) row[0] = 1.0f;
      if (k == 0) *reinterpret_cast<f2u*>(row + a.off1 + 2 * j) = f2u{S1.re, S1.im};
      float* r0 = row + a.off2 + (2 * j) * DIM + 2 * k;
      *reinterpret_cast<f2u*>(r0) = f2u{0.5f * (SA.re + SBv.re), 0.5f * (SBv.im - SA.im)};
      *reinterpret_cast<f2u*>(r0 + DIM) = f2u{0.5f * (SA.im + SBv.im), 0.5f * (SA.re - SBv.re)};
    }
  }
  S1d = dc{(double)S1.re, (double)S1.im};
  SAd = dc{(double)SA.re, (double)SA.im};
  SBd = dc{(double)SBv.re, (double)SBv.im};
}

template <bool BF16>
__global__ __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(3))) void k_fwd_lb(DiagArgs a) {
  constexpr int KP = 4, GPW = Geo<KP>::GPW;
  static_assert(GPW == 4, "one quad of chunks per workgroup");
  __shared__ __align__(16) float s_v[2][GPW * VBLK];
  __shared__ __align__(16) float s_row[GPW][RBUF];  // chunk summaries, then chunk carries, then row staging
  __shared__ dc s_F[GPW][K];                        // chunk flows
  __shared__ int s_tk, s_flag[GPW];
  __shared__ float s_hb[GPW];
  const int tid = threadIdx.x;
  const int NG = (a.NQ + LBG - 1) / LBG;
  const int b = blockIdx.x % a.B;  // consecutive workgroups take different samples
  if (tid == 0) s_tk = atomicAdd(a.lbflag + (size_t)a.B * (a.NQ + NG) + (size_t)b * LBT, 1);
  __syncthreads();
  const int q = s_tk;  // the sample's quads in the order its workgroups started
  const int cb = 4 * q, nc = min(GPW, a.C - cb);
  const Lane l = lane_of<KP>(tid);
  const int jj = tid >> 3, kk = tid & 7;
  const int c = cb + l.gi;
  const bool act = c < a.C;
  // ---- A: classification and chunk summaries from a zero state (the first chunk's operands of the closed form
  // and the table coefficients are loaded first: they do not depend on the classification)
  CfIn<BF16> in;
  lb_cf_load<BF16>(a, b, cb, in);
  const CfTab ct = cf_tab(a, jj, kk);
  int flag = 0;
  float hb = 0.0f;
  if (act) {
    flag = classify_chunk(a, b, c, l.gl, hb);
    if (l.gl == 0) {
      a.cflag[b * a.C + c] = flag;
      a.chbar[b * a.C + c] = hb;
      s_flag[l.gi] = flag;
      s_hb[l.gi] = hb;
    }
  }
  const bool quad_uni = __all(!act || (flag & 1));  // wavefront-uniform: the staging is shared
  const int t0 = act ? c * a.T : 0, Tc = act ? min(a.T, a.n_int - t0) : 0;
  if (quad_uni) {  // the summaries in closed form, chunk by chunk (lane = step); the next chunk's loads in flight
    __shared__ float s_tot[DIM];
    float(*s_x)[DIM] = reinterpret_cast<float(*)[DIM]>(&s_v[0][0]);  // the staging buffers are free here
    float(*s_y)[DIM] = reinterpret_cast<float(*)[DIM]>(&s_v[1][0]);
    __syncthreads();  // the groups' classifications
    CfIn<BF16> nx;
    for (int i = 0; i < nc; ++i) {
      if (i + 1 < nc) lb_cf_load<BF16>(a, b, cb + i + 1, nx);
      lb_summary_cf<BF16>(a, b, cb + i, s_hb[i], (s_flag[i] & 4) != 0, ct, in, s_x, s_y, s_tot, s_row[i]);
      in = nx;
    }
  } else {
    for (int i = 0; i < nc; ++i) {
      PairSt z{};
      lb_pairwise<false, BF16>(a, b, cb + i, jj, kk, z.S1, z.SA, z.SB);
      store_st_f(s_row[i], jj, kk, z);
    }
  }
  if (tid < 8 * nc) s_F[tid >> 3][tid & 7] = span_flow(a, b, cb + (tid >> 3), cb + (tid >> 3) + 1, tid & 7);
  __syncthreads();
  // ---- B: the quad's aggregate (lane = 8 jj + kk), published
  PairSt agg{};
  for (int i = 0; i < nc; ++i) {
    const float* sp = s_row[i];
    chen_d(agg, s_F[i][jj], s_F[i][kk], ld_fd(sp + 2 * jj), ld_fd(sp + 2 * kk), ld_fd(sp + poff(jj, kk)),
           ld_fd(sp + poff(jj, kk) + 2));
  }
  const dc qFj = span_flow(a, b, cb, cb + nc, jj), qFk = span_flow(a, b, cb, cb + nc, kk);
  const size_t AW = (size_t)a.D + 2 * K;
  LbItems it;
  it.qrow = a.lbagg + (size_t)b * a.NQ * AW;
  it.grow = a.lbagg + ((size_t)a.B * a.NQ + (size_t)b * NG) * AW;
  it.qst = a.lbflag + (size_t)b * a.NQ;
  it.gst = a.lbflag + (size_t)a.B * a.NQ + (size_t)b * NG;
  it.q = q;
  it.g = q / LBG;
  it.nq = q - LBG * it.g;
  it.ng = it.g;
  it.AW = AW;
  const bool last_of_group = it.nq == LBG - 1 && q + 1 < a.NQ;  // a later quad needs this group's aggregate
  publish(const_cast<double*>(it.qrow) + (size_t)q * AW, const_cast<int*>(it.qst) + q, a.D, jj, kk, agg, qFj);
  // ---- C: the carry: the group's earlier quads, then the earlier groups
  PairSt acc{};
  dc aFj{1.0, 0.0}, aFk{1.0, 0.0};
  // an aggregate still unpublished after kSpinLimit polls (a predecessor descheduled for that long) makes this
  // quad's carry, and through the published aggregates every later quad's, NaN: the rows show the failure
  const double qnan = __builtin_nan("");
  const PairSt poison{{qnan, qnan}, {qnan, qnan}, {qnan, qnan}};
  if (!lb_fold_ready(it, 0, it.nq, a.D, jj, kk, acc, aFj, aFk)) {
    acc = poison;
    lb_timeout(a);
  }
  if (last_of_group) {  // the group's aggregate: its earlier quads (folded) followed by this quad
    PairSt ga = acc;
    chen_d(ga, qFj, qFk, agg.S1, shfl_d(agg.S1, 8 * kk), agg.SA, agg.SB);
    publish(const_cast<double*>(it.grow) + (size_t)it.g * AW, const_cast<int*>(it.gst) + it.g, a.D, jj, kk, ga,
            aFj * qFj);
  }
  if (!lb_fold_ready(it, it.nq, it.nq + it.ng, a.D, jj, kk, acc, aFj, aFk)) {
    acc = poison;
    lb_timeout(a);
  }
  // ---- D: chunk carries inside the quad (for the backward), then the prefix rows
  {
    PairSt st = acc;  // the zero state followed by every earlier quad
    for (int i = 0; i < nc; ++i) {
      const float* sp = s_row[i];
      const PairSt y = load_st_f(sp, jj, kk);
      const dc y1k = ld_fd(sp + 2 * kk);
      __syncthreads();  // every lane has read summary i before the carry replaces it
      store_st_d(a.carries + ((size_t)b * (a.C + 1) + cb + i) * a.D, jj, kk, st);
      store_st_f(s_row[i], jj, kk, st);
      chen_d(st, s_F[i][jj], s_F[i][kk], y.S1, y1k, y.SA, y.SB);
    }
    if (cb + nc == a.C) store_st_d(a.carries + ((size_t)b * (a.C + 1) + a.C) * a.D, jj, kk, st);
  }
  __syncthreads();
  if (quad_uni) {
    FwdCoef<KP> f;
    fwd_coef<KP>(a, l, hb, (flag & 4) != 0, f);
    cf S1{0.0f, 0.0f}, SA[KP], SB_[KP];
    const float* cr = s_row[l.gi];
    S1 = cf{cr[2 * l.j], cr[2 * l.j + 1]};
    static_for<0, KP>([&](auto qc) {
      constexpr int qq = qc;
      const f4a p2 = *reinterpret_cast<const f4a*>(cr + poff(l.j, KP * l.kg + qq));
      SA[qq] = cf{0.5f * p2.x, 0.5f * p2.y};
      SB_[qq] = cf{0.5f * p2.z, 0.5f * p2.w};
    });
    wave_order();
    lb_steps<true, BF16>(a, l, b, cb, t0, Tc, f, S1, SA, SB_, s_v, s_row[l.gi]);
  } else {
    for (int i = 0; i < nc; ++i) {
      PairSt z = load_st_f(s_row[i], jj, kk);
      lb_pairwise<true, BF16>(a, b, cb + i, jj, kk, z.S1, z.SA, z.SB);
    }
  }
}

}  // namespace pairs

// ------------------------------------------------------------------------------------------------ host side
bool pairs_eligible(int structure, int depth, int dim, int readout, int flow_mode, int T) {
  return structure == EWS_STRUCT_PLANES && depth == 2 && dim == pairs::DIM && readout == EWS_READOUT_PREFIX &&
         flow_mode == EWS_FLOW_PER_INTERVAL && T <= kMaxT && T >= pairs::NB;
}

// out = false: the coefficient table (and the look-back words zeroed); out = true: the look-back forward (one
// workgroup per quad, tickets in launch order)
int pairs_forward(const DiagArgs& a, hipStream_t st, bool out) {
  if (!out) {
    // workgroup 0 the table, the others the aggregates' fill
    const size_t n = (size_t)a.B * (a.NQ + (a.NQ + pairs::LBG - 1) / pairs::LBG) * (a.D + 2 * pairs::K);
    const unsigned fill = (unsigned)std::min<size_t>(512, (n + 192 * 8 - 1) / (192 * 8));
    hipLaunchKernelGGL(pairs::k_coef_table, dim3(1 + fill), dim3(192), 0, st, a);
  } else {
    const dim3 grid(a.NQ * a.B), blk(64);
    if (a.path_bf16) hipLaunchKernelGGL((pairs::k_fwd_lb<true>), grid, blk, 0, st, a);
    else hipLaunchKernelGGL((pairs::k_fwd_lb<false>), grid, blk, 0, st, a);
  }
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

int pairs_carry_scan(const DiagArgs& a, hipStream_t st) {
  // the scan workgroups stage a segment of quads in more LDS than a static allocation may hold
  if (hipFuncSetAttribute(reinterpret_cast<const void*>(&pairs::k_quad_bwd_scan),
                          hipFuncAttributeMaxDynamicSharedMemorySize, (int)pairs::kScanLds) != hipSuccess)
    return -1;
  hipLaunchKernelGGL(pairs::k_quad_bwd_agg, dim3(a.NQ, a.B), dim3(64), 0, st, a);
  if (hipGetLastError() != hipSuccess) return -1;
  hipLaunchKernelGGL(pairs::k_quad_bwd_scan, dim3(a.B), dim3(pairs::SW * 64), pairs::kScanLds, st, a);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

// Without the clock gradient (dclock null) an invertible uniform chunk's adjoint is split by linearity: the full
// per-step adjoint of its own rows (pass 0, k_bwd_full<.., BW_LOCAL>, which reads the cotangent rows once) and the
// closed-form part of the later chunks' cotangent (pass 2, k_bwd_carry). With the clock gradient, pass 0 computes
// mu only and pass 2 runs the full adjoint (k_bwd_full<.., BW_FULL>), reading the rows again.
int pairs_backward(const DiagArgs& a, hipStream_t st, bool full) {
  const bool split = a.dclock == nullptr;
  if (full) {
    if (split) {
      if (a.path_bf16) hipLaunchKernelGGL((pairs::k_bwd_carry<true>), dim3(a.C, a.B), dim3(64), 0, st, a);
      else hipLaunchKernelGGL((pairs::k_bwd_carry<false>), dim3(a.C, a.B), dim3(64), 0, st, a);
    } else {
      constexpr int GPW = pairs::Geo<2>::GPW;
      const dim3 grid((a.C + GPW - 1) / GPW, a.B), blk(64);
      if (a.path_bf16) hipLaunchKernelGGL((pairs::k_bwd_full<true, true, pairs::BW_FULL>), grid, blk, 0, st, a);
      else hipLaunchKernelGGL((pairs::k_bwd_full<false, true, pairs::BW_FULL>), grid, blk, 0, st, a);
    }
  } else {
    constexpr int GPW = pairs::Geo<4>::GPW;
    const dim3 grid((a.C + GPW - 1) / GPW, a.B), blk(64);
    if (split) {
      if (a.path_bf16) hipLaunchKernelGGL((pairs::k_bwd_local<true, true>), grid, blk, 0, st, a);
      else hipLaunchKernelGGL((pairs::k_bwd_local<false, true>), grid, blk, 0, st, a);
      if (hipGetLastError() != hipSuccess) return -1;
      constexpr int GPW2 = pairs::Geo<2>::GPW;
      const dim3 grid2((a.C + GPW2 - 1) / GPW2, a.B);
      if (a.path_bf16) hipLaunchKernelGGL((pairs::k_bwd_full<true, false, pairs::BW_LOCAL>), grid2, blk, 0, st, a);
      else hipLaunchKernelGGL((pairs::k_bwd_full<false, false, pairs::BW_LOCAL>), grid2, blk, 0, st, a);
    } else {
      if (a.path_bf16) hipLaunchKernelGGL((pairs::k_bwd_local<true, false>), grid, blk, 0, st, a);
      else hipLaunchKernelGGL((pairs::k_bwd_local<false, false>), grid, blk, 0, st, a);
    }
  }
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // namespace ews
