// Token-cached scan at depth 1 for cached flows of any width up to 64 (ews/core/token_scan.py:91-118 with trunc 1):
// S_t = D_{g_t} S_{t-1} + P_{g_t} from S = 0, a padded step keeping the state (D = I, P = 0). D_cache (V, d, d) is a
// dense flow per token, P_cache (V, d) the token's level 1.
//
// Forward: one wavefront per sample, lane i the state coordinate i; a step reads the token's transposed flow (a
// transposed copy made first, so that lane i reads D[g][i][j] for fixed j from consecutive addresses) against the
// previous state broadcast through LDS. Backward: one wavefront per sample walks the steps in reverse,
// lam_t = g_t + D_{t+1}^T lam_{t+1} (lane j reads row i of D[g] contiguously), and stores every step's cotangent;
// then per token dP_g = sum lam_t and dD_g = sum lam_t S_{t-1}^T over the steps carrying it, from the forward's rows
// (the states), in per-chunk partials reduced in a fixed order (deterministic).
#include <hip/hip_runtime.h>

#include "ews_hip.h"
#include "ews_lanes.h"

namespace ews {
namespace tok1 {

constexpr int kMaxD = 64;
constexpr int kChunk = 2048;  // steps per partial of the token gradients
constexpr int kStage = 16;    // steps staged in LDS at once

struct TArgs {
  int B, n, d, V;
  const int32_t* tokens;  // (B, n)
  const uint8_t* mask;    // (B, n) or null
  const float* P;         // (V, d)
  const float* D;         // (V, d, d)
  float* Dt;              // (V, d, d) transposed copy (workspace)
  float* out;             // (B, n, d)
  const float* rows;      // the forward's rows (backward)
  const float* gout;      // (B, n, d)
  float* lam;             // (B, n, d) cotangent of every step's state (workspace)
  float* part;            // (V, nch, d*d + d) per-chunk partials (workspace)
  int nch;
  float* gP;
  float* gD;
};

__device__ __forceinline__ int tok_at(const TArgs& a, size_t e, bool& live) {
  live = a.mask == nullptr || a.mask[e] != 0;
  const int g = a.tokens[e];
  return g < 0 ? 0 : (g >= a.V ? a.V - 1 : g);
}

__global__ void k_transpose(TArgs a) {
  const size_t e = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  const size_t dd = (size_t)a.d * a.d;
  if (e >= (size_t)a.V * dd) return;
  const size_t g = e / dd, r = e % dd, i = r / a.d, j = r % a.d;
  a.Dt[g * dd + j * a.d + i] = a.D[e];
}

__global__ __launch_bounds__(64) void k_fwd(TArgs a) {
  __shared__ float s_x[kMaxD];
  const int b = blockIdx.x, i = threadIdx.x;
  const bool on = i < a.d;
  float S = 0.0f;
  for (int t = 0; t < a.n; ++t) {
    const size_t e = (size_t)b * a.n + t;
    bool live;
    const int g = tok_at(a, e, live);
    if (on) s_x[i] = S;
    __syncthreads();
    if (live && on) {
      const float* dt = a.Dt + (size_t)g * a.d * a.d + i;  // Dt[g][j][i] = D[g][i][j]
      float acc = a.P[(size_t)g * a.d + i];
      for (int j = 0; j < a.d; ++j) acc = fmaf(dt[(size_t)j * a.d], s_x[j], acc);
      S = acc;
    }
    if (on) a.out[e * a.d + i] = S;
    __syncthreads();  // s_x is rewritten by the next step
  }
}

__global__ __launch_bounds__(64) void k_bwd_lam(TArgs a) {
  __shared__ float s_l[kMaxD];
  const int b = blockIdx.x, j = threadIdx.x;
  const bool on = j < a.d;
  float lam = 0.0f;
  for (int t = a.n - 1; t >= 0; --t) {
    const size_t e = (size_t)b * a.n + t;
    if (on) {
      lam += a.gout[e * a.d + j];
      a.lam[e * a.d + j] = lam;
      s_l[j] = lam;
    }
    __syncthreads();
    bool live;
    const int g = tok_at(a, e, live);
    if (live && on) {  // lam_{t-1} carried = D_g^T lam_t: lane j takes column j (row i contiguous over lanes)
      const float* dg = a.D + (size_t)g * a.d * a.d + j;
      float acc = 0.0f;
      for (int i = 0; i < a.d; ++i) acc = fmaf(dg[(size_t)i * a.d], s_l[i], acc);
      lam = acc;
    }
    __syncthreads();
  }
}

// partials of token g over steps [c * kChunk, (c + 1) * kChunk) of the flattened (sample, step) order: each thread
// owns 16 entries of dD_g (d <= 64), threads < d also an entry of dP_g
__global__ __launch_bounds__(256) void k_grads(TArgs a) {
  __shared__ float s_l[kStage][kMaxD], s_s[kStage][kMaxD];
  __shared__ int s_use[kStage];
  const int g = blockIdx.x, c = blockIdx.y, tid = threadIdx.x;
  const size_t tot = (size_t)a.B * a.n, e0 = (size_t)c * kChunk, e1 = min(tot, e0 + kChunk);
  const int dd = a.d * a.d;
  float acc[16], accp = 0.0f;
#pragma unroll
  for (int k = 0; k < 16; ++k) acc[k] = 0.0f;
  for (size_t s0 = e0; s0 < e1; s0 += kStage) {
    // stage the block's steps that carry token g: their cotangents and the states before them
    for (int q = tid; q < kStage * kMaxD; q += 256) {
      const int r = q / kMaxD, col = q % kMaxD;
      const size_t e = s0 + r;
      bool use = false;
      if (e < e1) {
        bool live;
        use = tok_at(a, e, live) == g && live;
      }
      if (col == 0) s_use[r] = use;
      float lv = 0.0f, sv = 0.0f;
      if (use && col < a.d) {
        lv = a.lam[e * a.d + col];
        const size_t t = e % a.n;
        sv = t > 0 ? a.rows[(e - 1) * a.d + col] : 0.0f;  // S_{t-1} (zero before the first step)
      }
      s_l[r][col] = lv;
      s_s[r][col] = sv;
    }
    __syncthreads();
    for (int r = 0; r < kStage; ++r) {
      if (!s_use[r]) continue;  // uniform across the workgroup
#pragma unroll
      for (int k = 0; k < 16; ++k) {
        const int q = tid + 256 * k;
        if (q < dd) acc[k] = fmaf(s_l[r][q / a.d], s_s[r][q % a.d], acc[k]);
      }
      if (tid < a.d) accp += s_l[r][tid];
    }
    __syncthreads();
  }
  float* out = a.part + ((size_t)g * a.nch + c) * (dd + a.d);
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    const int q = tid + 256 * k;
    if (q < dd) out[q] = acc[k];
  }
  if (tid < a.d) out[dd + tid] = accp;
}

// the chunks' partials summed in order, float64
__global__ void k_reduce(TArgs a) {
  const int dd = a.d * a.d, W = dd + a.d;
  const size_t e = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= (size_t)a.V * W) return;
  const size_t g = e / W, q = e % W;
  double s = 0.0;
  for (int c = 0; c < a.nch; ++c) s += (double)a.part[((size_t)g * a.nch + c) * W + q];
  if ((int)q < dd) a.gD[g * dd + q] = (float)s;
  else a.gP[g * a.d + (q - dd)] = (float)s;
}

// ---- block-diagonal caches (desc->block = BS): the flow of every token is block-diagonal with blocks of BS
// consecutive coordinates (the chain-structured caches: rotation planes BS = 2, Jordan chains BS = their size, a
// real diagonal BS = 1). Lane i then needs only row i of its block: S_i = P_g[i] + sum_r D_g[i][base + r] S_{base+r}
// (base = BS floor(i / BS)), with the block partners' states by lane shuffles: no LDS broadcast, no barrier. The
// caches' block entries are staged in LDS when they fit (row i of token g's block at (g d + i) BS), the step's token
// and mask bit come from a register holding the next 64 steps. The backward walks the steps in reverse with the
// cotangent lam_{t-1} = D_g^T lam_t (+ the row cotangent), and accumulates the token gradients per lane in LDS
// (lane i owns dP_g[i] and row i of dD_g's block): per-sample partials, then a fixed-order sum over the samples.
// Entries of D outside the blocks are taken as zero and their gradients are written as zero.
constexpr int kStageFloats = 12288;  // caches staged in LDS up to 48 KB

template <bool STAGED>
__device__ __forceinline__ float blk_d(const TArgs& a, const float* sD, int BS, int g, int row, int r) {
  if constexpr (STAGED) return sD[((size_t)g * a.d + row) * BS + r];
  return a.D[((size_t)g * a.d + row) * a.d + (row / BS) * BS + r];
}

// v of lane base + r, the r-th lane of this lane's block (base = BS floor(lane / BS)); every lane of the wavefront
// takes part. Blocks of 2 and 4 lie inside a quad of lanes: one DPP quad permutation (a VALU operand, no memory
// round trip); blocks of 3, 6 and 8 go through an LDS permute.
template <int BS>
__device__ __forceinline__ float blk_lane(float v, int base, int r) {
  if constexpr (BS == 1) {
    return v;
  } else if constexpr (BS == 2) {
    return r == 0 ? lanes::dpp<0xA0>(v) : lanes::dpp<0xF5>(v);  // quad_perm [0, 0, 2, 2], [1, 1, 3, 3]
  } else if constexpr (BS == 4) {
    switch (r) {  // quad_perm [r, r, r, r]
      case 0: return lanes::dpp<0x00>(v);
      case 1: return lanes::dpp<0x55>(v);
      case 2: return lanes::dpp<0xAA>(v);
      default: return lanes::dpp<0xFF>(v);
    }
  } else {
    return __shfl(v, base + r);
  }
}

// the block caches into LDS (row i of token g's block at (g d + i) BS, then P), eight loads in flight per lane
template <int BS>
__device__ __forceinline__ void stage_blk(const TArgs& a, float* sP, float* sD, bool with_p, int i) {
  const int nd = a.V * a.d * BS;
  for (int q0 = i; q0 < nd; q0 += 8 * 64) {
    float v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int q = min(q0 + 64 * u, nd - 1);  // clamped: every load unconditional
      const int gr = q / BS, r = q - gr * BS, g = gr / a.d, row = gr - g * a.d;
      v[u] = a.D[((size_t)g * a.d + row) * a.d + (row / BS) * BS + r];
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      if (q0 + 64 * u < nd) sD[q0 + 64 * u] = v[u];
    }
  }
  if (with_p) {
    const int np = a.V * a.d;
    for (int q0 = i; q0 < np; q0 += 8 * 64) {
      float v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) v[u] = a.P[min(q0 + 64 * u, np - 1)];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        if (q0 + 64 * u < np) sP[q0 + 64 * u] = v[u];
      }
    }
  }
}

// The step loops take the caches from LDS (STAGED) or from global memory, a compile-time choice: one load kind each
template <int BS, bool STAGED>
__device__ __forceinline__ void fwd_blk_steps(const TArgs& a, const float* sP, const float* sD, int b, int i) {
  const bool on = i < a.d;
  const int base = (i / BS) * BS;
  const int row = on ? i : 0;  // lanes past d read row 0 and keep S = 0
  float S = 0.0f;
  for (int t0 = 0; t0 < a.n; t0 += 64) {
    int tokv = 0, livev = 0;
    if (t0 + i < a.n) {
      bool live;
      tokv = tok_at(a, (size_t)b * a.n + t0 + i, live);
      livev = live ? 1 : 0;
    }
    const int cnt = min(64, a.n - t0);
    // groups of eight steps without a branch (the lane reads are convergent, so only a constant trip count is
    // unrolled; the states are stored after the group), so that the group's cache reads are issued ahead of the
    // state chain; steps past n carry token 0 and no mask bit
    for (int s0 = 0; s0 < 64; s0 += 8) {
      float Sv[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int g = __builtin_amdgcn_readlane(tokv, s0 + u), live = __builtin_amdgcn_readlane(livev, s0 + u);
        float acc = STAGED ? sP[g * a.d + row] : a.P[(size_t)g * a.d + row];
        float dr[BS];
#pragma unroll
        for (int r = 0; r < BS; ++r) dr[r] = blk_d<STAGED>(a, sD, BS, g, row, r);
#pragma unroll
        for (int r = 0; r < BS; ++r) acc = fmaf(dr[r], blk_lane<BS>(S, base, r), acc);
        if (live && on) S = acc;
        Sv[u] = S;
      }
      if (on) {
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          if (s0 + u < cnt) a.out[((size_t)b * a.n + t0 + s0 + u) * a.d + i] = Sv[u];
        }
      }
    }
  }
}

template <int BS>
__global__ __launch_bounds__(64) void k_fwd_blk(TArgs a) {
  extern __shared__ float s_c[];
  const int b = blockIdx.x, i = threadIdx.x;
  float* sP = s_c;
  float* sD = s_c + (size_t)a.V * a.d;
  if ((size_t)a.V * a.d * (BS + 1) <= (size_t)kStageFloats) {
    stage_blk<BS>(a, sP, sD, true, i);
    __syncthreads();
    fwd_blk_steps<BS, true>(a, sP, sD, b, i);
  } else {
    fwd_blk_steps<BS, false>(a, sP, sD, b, i);
  }
}

template <int BS, bool STAGED>
__device__ __forceinline__ void bwd_blk_steps(const TArgs& a, const float* sD, float* sAcc, float* sG, float* sR,
                                              int b, int i) {
  const bool on = i < a.d;
  const int base = (i / BS) * BS;
  // lanes past d read block row 0 (their products are dropped); their lam, state and accumulators stay zero
  const int rowb = on ? base : 0, col = on ? i - base : 0, ic = on ? i : 0;
  float lam = 0.0f;
  for (int t1 = a.n; t1 > 0; t1 -= 64) {
    const int t0 = max(0, t1 - 64);
    int tokv = 0, livev = 0;
    if (t0 + i < t1) {
      bool live;
      tokv = tok_at(a, (size_t)b * a.n + t0 + i, live);
      livev = live ? 1 : 0;
    }
    for (int u1 = t1; u1 > t0; u1 -= kStage) {
      const int u0 = max(t0, u1 - kStage);
      {  // the stage's inputs: unconditional loads from clamped (valid) addresses, all issued before the first
         // store, zeroed afterwards
        float gv[kStage], rv[kStage];
#pragma unroll
        for (int k = 0; k < kStage; ++k) {
          const int t = min(u0 + k, u1 - 1), tp = max(t - 1, 0);
          gv[k] = a.gout[((size_t)b * a.n + t) * a.d + ic];
          rv[k] = a.rows[((size_t)b * a.n + tp) * a.d + ic];  // S_{t-1}
        }
#pragma unroll
        for (int k = 0; k < kStage; ++k) {
          const int t = u0 + k;
          sG[k * 64 + i] = (on && t < u1) ? gv[k] : 0.0f;
          sR[k * 64 + i] = (on && t < u1 && t > 0) ? rv[k] : 0.0f;
        }
      }
      // steps u1 - 1 down to u0, unrolled and without a branch (see the forward): a step past u1 or without its
      // mask bit adds zero to the accumulators (exact: they start at +0 and never become -0) and keeps lam
#pragma unroll
      for (int k = kStage - 1; k >= 0; --k) {
        const int t = u0 + k;  // t - t0 < 64
        // uniform over the wavefront: the step's token and mask bit from lane t - t0
        const int g = __builtin_amdgcn_readlane(tokv, t - t0);
        const bool live = __builtin_amdgcn_readlane(livev, t - t0) && t < u1;
        lam += sG[k * 64 + i];
        const float sp = sR[k * 64 + i];
        const float lw = live ? lam : 0.0f;
        float* acc = sAcc + (size_t)g * (BS + 1) * 64 + i;
        float ln = 0.0f;
#pragma unroll
        for (int r = 0; r < BS; ++r) {
          const float s_r = blk_lane<BS>(sp, base, r), l_r = blk_lane<BS>(lam, base, r);
          acc[r * 64] += lw * s_r;                                              // dD_g[i][base + r]
          ln = fmaf(blk_d<STAGED>(a, sD, BS, g, rowb + r, col), l_r, ln);       // (D_g^T lam)_i
        }
        acc[BS * 64] += lw;  // dP_g[i]
        lam = live ? (on ? ln : 0.0f) : lam;
      }
    }
  }
}

template <int BS>
__global__ __launch_bounds__(64) void k_bwd_blk(TArgs a) {
  extern __shared__ float s_c[];
  const int b = blockIdx.x, i = threadIdx.x;
  const bool on = i < a.d;
  const bool staged = (size_t)a.V * a.d * (BS + 1) <= (size_t)kStageFloats;
  float* sD = s_c + (size_t)a.V * a.d;  // the same layout as the forward's (P's slot unused)
  float* sAcc = staged ? sD + (size_t)a.V * a.d * BS : s_c;  // (V, BS + 1, 64): lane i's column
  // kStage steps' row cotangents and previous states, lane i's column of each (only lane i reads it: no barrier)
  float* sG = sAcc + (size_t)a.V * (BS + 1) * 64;
  float* sR = sG + kStage * 64;
  if (staged) stage_blk<BS>(a, nullptr, sD, false, i);
  for (int q = 0; q < a.V * (BS + 1); ++q) sAcc[q * 64 + i] = 0.0f;
  __syncthreads();
  if (staged) bwd_blk_steps<BS, true>(a, sD, sAcc, sG, sR, b, i);
  else bwd_blk_steps<BS, false>(a, sD, sAcc, sG, sR, b, i);
  if (on) {
    for (int q = 0; q < a.V * (BS + 1); ++q)
      a.part[(((size_t)b * a.V * (BS + 1)) + q) * a.d + i] = sAcc[q * 64 + i];
  }
}

// gP and gD from the per-sample partials (samples in order, float64); gD's entries outside the blocks are zero
__global__ void k_reduce_blk(TArgs a, int BS) {
  const size_t e = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  const size_t dd = (size_t)a.d * a.d, tot = (size_t)a.V * (dd + a.d);
  if (e >= tot) return;
  int g, i, r;
  bool isP;
  if (e < (size_t)a.V * dd) {
    g = (int)(e / dd);
    const int rc = (int)(e - (size_t)g * dd);
    i = rc / a.d;
    const int col = rc - i * a.d;
    r = col - (i / BS) * BS;
    isP = false;
    if (r < 0 || r >= BS) {
      a.gD[e] = 0.0f;
      return;
    }
  } else {
    const size_t q = e - (size_t)a.V * dd;
    g = (int)(q / a.d);
    i = (int)(q - (size_t)g * a.d);
    r = BS;
    isP = true;
  }
  // the samples in order; eight loads in flight before their adds (the same order of additions)
  const size_t off = ((size_t)g * (BS + 1) + r) * a.d + i, stride = (size_t)a.V * (BS + 1) * a.d;
  double s = 0.0;
  int b = 0;
  for (; b + 8 <= a.B; b += 8) {
    float v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) v[u] = a.part[(size_t)(b + u) * stride + off];
#pragma unroll
    for (int u = 0; u < 8; ++u) s += (double)v[u];
  }
  for (; b < a.B; ++b) s += (double)a.part[(size_t)b * stride + off];
  if (isP) a.gP[(size_t)g * a.d + i] = (float)s;
  else a.gD[e] = (float)s;
}

}  // namespace tok1

namespace {
int tok1_check(const ews_token1_desc* s) {
  if (!s) return EWS_ERR_NULL;
  if (s->batch < 1 || s->steps < 1 || s->dim < 1 || s->dim > tok1::kMaxD || s->vocab < 1) return EWS_ERR_SHAPE;
  const int bs = s->block;
  if (bs < 0 || bs > 8 || bs == 5 || bs == 7 || (bs > 0 && s->dim % bs != 0)) return EWS_ERR_OPTION;
  // the backward's per-lane accumulators (16 KB at most) and its staged steps (8 KB) sit in LDS beside the staged
  // caches (48 KB at most)
  if (bs > 0 && (size_t)s->vocab * (bs + 1) > 64) return EWS_ERR_SHAPE;
  return EWS_OK;
}
// launch of a block-diagonal kernel for the descriptor's block size
#define EWS_TOK1_BLK(KERNEL, BS, GRID, LDS, ST, A)                                                    \
  do {                                                                                               \
    switch (BS) {                                                                                    \
      case 1: hipLaunchKernelGGL((KERNEL<1>), GRID, dim3(64), LDS, ST, A); break;                  \
      case 2: hipLaunchKernelGGL((KERNEL<2>), GRID, dim3(64), LDS, ST, A); break;                  \
      case 3: hipLaunchKernelGGL((KERNEL<3>), GRID, dim3(64), LDS, ST, A); break;                  \
      case 4: hipLaunchKernelGGL((KERNEL<4>), GRID, dim3(64), LDS, ST, A); break;                  \
      case 6: hipLaunchKernelGGL((KERNEL<6>), GRID, dim3(64), LDS, ST, A); break;                  \
      default: hipLaunchKernelGGL((KERNEL<8>), GRID, dim3(64), LDS, ST, A); break;                 \
    }                                                                                                \
  } while (0)
size_t blk_lds_bytes(const ews_token1_desc* s, bool bwd) {
  const size_t stage = (size_t)s->vocab * s->dim * (s->block + 1);
  const size_t staged = stage <= (size_t)tok1::kStageFloats ? stage : 0;
  return (staged + (bwd ? (size_t)s->vocab * (s->block + 1) * 64 + 2 * tok1::kStage * 64 : 0)) * 4;
}
size_t al256t(size_t x) { return (x + 255) & ~(size_t)255; }
tok1::TArgs tok1_args(const ews_token1_desc* s) {
  tok1::TArgs a{};
  a.B = s->batch;
  a.n = s->steps;
  a.d = s->dim;
  a.V = s->vocab;
  a.nch = (int)(((size_t)a.B * a.n + tok1::kChunk - 1) / tok1::kChunk);
  return a;
}
}  // namespace
}  // namespace ews

extern "C" {

size_t ews_token1_workspace_bytes(const ews_token1_desc* desc) {
  if (ews::tok1_check(desc) != EWS_OK) return 0;
  const ews::tok1::TArgs a = ews::tok1_args(desc);
  if (desc->block > 0) return ews::al256t((size_t)a.B * a.V * (desc->block + 1) * a.d * 4);  // per-sample partials
  const size_t dd = (size_t)a.d * a.d;
  return ews::al256t((size_t)a.V * dd * 4) + ews::al256t((size_t)a.B * a.n * a.d * 4) +
         ews::al256t((size_t)a.V * a.nch * (dd + a.d) * 4);
}

int ews_token1_scan(const ews_token1_desc* desc, const int32_t* tokens, const uint8_t* mask, const float* P_cache,
                    const float* D_cache, float* out, void* workspace, ews_stream_t stream) {
  const int rc = ews::tok1_check(desc);
  if (rc != EWS_OK) return rc;
  if (!tokens || !P_cache || !D_cache || !out || !workspace) return EWS_ERR_NULL;
  ews::tok1::TArgs a = ews::tok1_args(desc);
  a.tokens = tokens;
  a.mask = mask;
  a.P = P_cache;
  a.D = D_cache;
  a.Dt = (float*)workspace;
  a.out = out;
  hipStream_t st = (hipStream_t)stream;
  if (desc->block > 0) {
    EWS_TOK1_BLK(ews::tok1::k_fwd_blk, desc->block, dim3(a.B), ews::blk_lds_bytes(desc, false), st, a);
    return hipGetLastError() == hipSuccess ? EWS_OK : EWS_ERR_LAUNCH;
  }
  const size_t nd = (size_t)a.V * a.d * a.d;
  hipLaunchKernelGGL(ews::tok1::k_transpose, dim3((unsigned)((nd + 255) / 256)), dim3(256), 0, st, a);
  if (hipGetLastError() != hipSuccess) return EWS_ERR_LAUNCH;
  hipLaunchKernelGGL(ews::tok1::k_fwd, dim3(a.B), dim3(64), 0, st, a);
  return hipGetLastError() == hipSuccess ? EWS_OK : EWS_ERR_LAUNCH;
}

int ews_token1_scan_backward(const ews_token1_desc* desc, const int32_t* tokens, const uint8_t* mask,
                             const float* P_cache, const float* D_cache, const float* out, const float* grad_out,
                             float* grad_P, float* grad_D, void* workspace, ews_stream_t stream) {
  const int rc = ews::tok1_check(desc);
  if (rc != EWS_OK) return rc;
  if (!tokens || !P_cache || !D_cache || !out || !grad_out || !grad_P || !grad_D || !workspace) return EWS_ERR_NULL;
  ews::tok1::TArgs a = ews::tok1_args(desc);
  a.tokens = tokens;
  a.mask = mask;
  a.P = P_cache;
  a.D = D_cache;
  a.rows = out;
  a.gout = grad_out;
  a.gP = grad_P;
  a.gD = grad_D;
  const size_t dd = (size_t)a.d * a.d;
  hipStream_t st = (hipStream_t)stream;
  if (desc->block > 0) {
    a.part = (float*)workspace;
    EWS_TOK1_BLK(ews::tok1::k_bwd_blk, desc->block, dim3(a.B), ews::blk_lds_bytes(desc, true), st, a);
    if (hipGetLastError() != hipSuccess) return EWS_ERR_LAUNCH;
    const size_t tot = (size_t)a.V * (dd + a.d);
    hipLaunchKernelGGL(ews::tok1::k_reduce_blk, dim3((unsigned)((tot + 255) / 256)), dim3(256), 0, st, a,
                       desc->block);
    return hipGetLastError() == hipSuccess ? EWS_OK : EWS_ERR_LAUNCH;
  }
  char* w = (char*)workspace;
  a.lam = (float*)(w + ews::al256t((size_t)a.V * dd * 4));
  a.part = (float*)(w + ews::al256t((size_t)a.V * dd * 4) + ews::al256t((size_t)a.B * a.n * a.d * 4));
  hipLaunchKernelGGL(ews::tok1::k_bwd_lam, dim3(a.B), dim3(64), 0, st, a);
  if (hipGetLastError() != hipSuccess) return EWS_ERR_LAUNCH;
  hipLaunchKernelGGL(ews::tok1::k_grads, dim3(a.V, a.nch), dim3(256), 0, st, a);
  if (hipGetLastError() != hipSuccess) return EWS_ERR_LAUNCH;
  const size_t W = (size_t)a.V * (dd + a.d);
  hipLaunchKernelGGL(ews::tok1::k_reduce, dim3((unsigned)((W + 255) / 256)), dim3(256), 0, st, a);
  return hipGetLastError() == hipSuccess ? EWS_OK : EWS_ERR_LAUNCH;
}

}  // extern "C"
