// Mixer epilogue of an EWS block on MI355X (gfx950), fused: the prefix rows' levels without their level-0
// column, an optional leading zero row, the optional binomial prescale, the per-level GradedRMSNorm and the
// c_down linear map, in one pass over the D-wide rows. Only the hidden-wide output is written.
//
// Reference (ews/block.py:282-306, 336-357, 405-408; ews/norms.py:47-134):
//   levels = flat[:, 1:] (with a zero row in front unless basepoint), z_k = c(t, k) levels_k (binomial prescale,
//   c = 1 / C(max(t_len, k), k), t_len = levels row + 1, or 1), y_k = s_k z_k with
//     live_rms    s_k = g_k / (RMS(z_k) + eps_k)   (RMS over the level's d^k coordinates; 0 for an all-zero level)
//     static_gain s_k = g_k
//     dilation    s_k = lam^k,
//   r = W y + b (eqx.nn.Linear(D, hidden)).
// Since every scale is one number per row and level, r = b + sum_k f_k P_k with P_k = W_k x_k (W_k the level's
// column block, x the unscaled row) and f_k = s_k c: the kernel accumulates P_k and the level's sum of squares in
// one pass and applies f_k at the end.
//
// Backward (dr = dL/dr): dx_k = f_k W_k^T dr - beta_k (P_k . dr) x_k, with beta_k = g_k c^2 / ((c rho + eps)^2
// n rho), rho = RMS(x_k), n = d^k, for live_rms (0 at rho = 0, where the reference's RMS has a zero gradient),
// beta = 0 otherwise. The parameter gradients need only row-level quantities (host side).
//
// MFMA: v_mfma_f32_16x16x4f32 (lane l: A[l%16][l/16], B[l/16][l%16], result rows 4(l/16)+r of column l%16). The
// contraction index of each 16-wide block is permuted so that a lane's four k-steps read four consecutive floats
// of its row (slot g of step s is k0 + 4g + s), which changes nothing in the sum.
#include <hip/hip_runtime.h>

#include <cmath>
#include <type_traits>

#include "ews_hip.h"
#include "ews_lanes.h"

namespace ews {
namespace mixer {

typedef float f4 __attribute__((ext_vector_type(4)));
typedef float f4u __attribute__((ext_vector_type(4), aligned(4)));

struct MArgs {
  int B, R, d, N, lvl0, W, D, hidden, variant, prepend, prescale;
  float eps[3];
  int st[3], n[3];  // level offsets (level-0-free) and sizes
  const float* rows;
  const float* weight;
  const float* bias;
  const float* gains;
  float* out;
  float* P;  // (B R, N, hidden) level products
  float* F;  // (B R, N, 3): total scale f, beta, d f / d gain
  const float* gout;
  float* grows;
  float* dots;  // (B R, N)
  float* dwpart;  // (row chunks, hidden, D) partial c_down weight gradients of the column kernel
};

__device__ __forceinline__ f4 mfma(float a, float b, f4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// p[k .. k+3] of a run ending at `end` (entries at or past end read as zero); nothing is read when !ok
__device__ __forceinline__ f4 load4(const float* p, int k, int end, bool ok) {
  if (!ok) return f4{0.0f, 0.0f, 0.0f, 0.0f};
  if (k + 3 < end) {
    const f4u v = *reinterpret_cast<const f4u*>(p + k);
    return f4{v.x, v.y, v.z, v.w};
  }
  return f4{k < end ? p[k] : 0.0f, k + 1 < end ? p[k + 1] : 0.0f, k + 2 < end ? p[k + 2] : 0.0f,
            k + 3 < end ? p[k + 3] : 0.0f};
}

// orders a wavefront's LDS accesses across lanes: no access moves across it (the hardware keeps a wavefront's LDS
// operations in program order)
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

template <int I, int N, class Fn> __device__ __forceinline__ void sfor(Fn&& f) {
  if constexpr (I < N) {
    f(std::integral_constant<int, I>{});
    sfor<I + 1, N>(f);
  }
}

// output row of scan row gr (sample b, row t)
__device__ __forceinline__ size_t out_row(const MArgs& a, int gr) {
  const int b = gr / a.R, t = gr - b * a.R;
  return (size_t)b * (a.R + a.prepend) + t + a.prepend;
}

// Forward: a workgroup = 4 wavefronts x RT tiles of 16 rows, hidden columns [16 NH blockIdx.y, +16 NH). The RT
// row tiles of a wavefront share each load of c_down's rows.
template <int N, int NH, int RT>
__global__ __launch_bounds__(256) void k_mix_fwd(MArgs a) {
  __shared__ float s_f[4][RT][3][16];
  const int w = threadIdx.x >> 6, l = threadIdx.x & 63, i = l & 15, g = l >> 4;
  const int M = a.B * a.R;
  const int row0 = (blockIdx.x * 4 + w) * 16 * RT;
  const int hc = blockIdx.y * 16 * NH;
  const float* xp[RT];
  bool valid[RT];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    const int gr = row0 + 16 * rt + i;
    valid[rt] = gr < M;
    xp[rt] = a.rows + (size_t)(valid[rt] ? gr : 0) * a.W + a.lvl0;
  }
  f4 acc[N][NH][RT];
  float ssq[N][RT];
  sfor<0, N>([&](auto kc) {
    constexpr int k = kc;
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      ssq[k][rt] = 0.0f;
#pragma unroll
      for (int h = 0; h < NH; ++h) acc[k][h][rt] = f4{0.0f, 0.0f, 0.0f, 0.0f};
    }
  });
  sfor<0, N>([&](auto kc) {
    constexpr int k = kc;
    const int st = a.st[k], en = st + a.n[k];
    for (int k0 = st; k0 < en; k0 += 16) {
      const int kk = k0 + 4 * g;
      f4 xa[RT];
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) {
        xa[rt] = load4(xp[rt], kk, en, valid[rt]);
        ssq[k][rt] = fmaf(xa[rt].x, xa[rt].x,
                          fmaf(xa[rt].y, xa[rt].y, fmaf(xa[rt].z, xa[rt].z, fmaf(xa[rt].w, xa[rt].w, ssq[k][rt]))));
      }
#pragma unroll
      for (int h = 0; h < NH; ++h) {
        const int hrow = hc + 16 * h + i;
        const bool hok = hrow < a.hidden;
        const f4 wb = load4(a.weight + (size_t)(hok ? hrow : 0) * a.D, kk, en, hok);
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
          acc[k][h][rt] = mfma(xa[rt].x, wb.x, acc[k][h][rt]);
          acc[k][h][rt] = mfma(xa[rt].y, wb.y, acc[k][h][rt]);
          acc[k][h][rt] = mfma(xa[rt].z, wb.z, acc[k][h][rt]);
          acc[k][h][rt] = mfma(xa[rt].w, wb.w, acc[k][h][rt]);
        }
      }
    }
  });
  // per-row factors: the four lanes of a row hold partial sums of squares
  sfor<0, N>([&](auto kc) {
    constexpr int k = kc;
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      float v = ssq[k][rt];
      v = lanes::add_xor32(lanes::add_xor16(v));
      if (g == 0) {
        const int gr = row0 + 16 * rt + i;
        const int t = valid[rt] ? gr % a.R : 0;
        const int K = k + 1;
        float c = 1.0f;
        if (a.prescale) {
          const double tl = fmax((double)(t + 1 + a.prepend), (double)K);
          c = (float)exp(-(lgamma(tl + 1.0) - lgamma(tl - K + 1.0) - lgamma((double)K + 1.0)));
        }
        float f, beta = 0.0f, dfdg;
        if (a.variant == EWS_GRADED_LIVE_RMS) {
          const float gk = a.gains[k];
          const float ms = v / (float)a.n[k];
          const float rho = ms > 0.0f ? sqrtf(ms) : 0.0f;
          const float den = fmaf(c, rho, a.eps[k]);
          dfdg = c / den;
          f = gk * dfdg;
          if (rho > 0.0f) beta = gk * c * c / (den * den * (float)a.n[k] * rho);
        } else if (a.variant == EWS_GRADED_STATIC_GAIN) {
          dfdg = c;
          f = a.gains[k] * c;
        } else {
          const float lam = a.gains[0];
          const float lk1 = powf(lam, (float)(K - 1));
          dfdg = (float)K * lk1 * c;
          f = lk1 * lam * c;
        }
        s_f[w][rt][k][i] = f;
        if (valid[rt] && blockIdx.y == 0) {
          float* fp = a.F + ((size_t)gr * N + k) * 3;
          fp[0] = f;
          fp[1] = beta;
          fp[2] = dfdg;
        }
      }
    }
  });
  __syncthreads();
#pragma unroll
  for (int h = 0; h < NH; ++h) {
    const int col = hc + 16 * h + i;
    if (col < a.hidden) {
      const float bc = a.bias[col];
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int row = 4 * g + r, grow = row0 + 16 * rt + row;
          if (grow < M) {
            float v = bc;
            sfor<0, N>([&](auto kc) {
              constexpr int k = kc;
              const f4 q = acc[k][h][rt];
              const float pv = r == 0 ? q.x : (r == 1 ? q.y : (r == 2 ? q.z : q.w));
              v = fmaf(s_f[w][rt][k][row], pv, v);
              a.P[((size_t)grow * N + k) * a.hidden + col] = pv;
            });
            a.out[out_row(a, grow) * a.hidden + col] = v;
          }
        }
      }
    }
  }
}

// Forward with streamed rows: a wavefront per RT tiles of 16 consecutive rows (one contiguous run of 16 RT W floats),
// all hidden columns (NH tiles of 16). Each level is walked in segments of SEG entries: the rows' segment is loaded
// with 16-byte loads (SEG / 4 lanes per row: runs of 4 SEG bytes) into the wavefront's LDS tile while the previous
// segment is contracted from it (the next segment's loads in flight in registers), then read in the MFMA layout;
// each c_down fragment serves the RT row tiles. The per-row factors are exchanged by lane shuffles, so nothing
// crosses wavefronts.
__device__ __forceinline__ f4 ld_seg4(const float* p, int c, int nc, bool ok) {
  // p[c .. c+3] of a run whose valid entries end at nc (dword-aligned; unaligned 16-byte loads are fine)
  if (!ok || c >= nc) return f4{0.0f, 0.0f, 0.0f, 0.0f};
  if (c + 3 < nc) {
    const f4u v = *reinterpret_cast<const f4u*>(p + c);
    return f4{v.x, v.y, v.z, v.w};
  }
  return f4{p[c], c + 1 < nc ? p[c + 1] : 0.0f, c + 2 < nc ? p[c + 2] : 0.0f, 0.0f};
}

template <int N, int NH, int RT>
__global__ __launch_bounds__(256) void k_mix_fwd_s(MArgs a) {
  constexpr int SEG = 128 / RT, PITCH = SEG + 4, RW = 16 * RT;  // 16-byte LDS rows, 4 banks apart
  constexpr int NV = RW * SEG / 4 / 64;                         // 16-byte loads per lane per segment
  __shared__ __align__(16) float s_x[4][RW][PITCH];
  const int w = threadIdx.x >> 6, l = threadIdx.x & 63, i = l & 15, g = l >> 4;
  const int M = a.B * a.R;
  const int row0 = (blockIdx.x * 4 + w) * RW;
  if (row0 >= M) return;  // uniform over the wavefront; no workgroup barrier below
  float(*sx)[PITCH] = s_x[w];
  f4 acc[N][NH][RT];
  float ssq[N][RT];
#pragma unroll
  for (int k = 0; k < N; ++k)
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      ssq[k][rt] = 0.0f;
#pragma unroll
      for (int h = 0; h < NH; ++h) acc[k][h][rt] = f4{0.0f, 0.0f, 0.0f, 0.0f};
    }
  // the (level, segment) walk: segment q of level k covers entries [st_k + SEG q, ...)
  auto seg_load = [&](int k, int q, f4 (&v)[NV]) {
    const int base = a.lvl0 + a.st[k] + SEG * q, nc = a.n[k] - SEG * q;
#pragma unroll
    for (int u = 0; u < NV; ++u) {
      const int e = l + 64 * u, r = e / (SEG / 4), c = 4 * (e % (SEG / 4)), gr = row0 + r;
      v[u] = ld_seg4(a.rows + (size_t)(gr < M ? gr : 0) * a.W + base, c, nc, gr < M);
    }
  };
  f4 nx[NV];
  int k = 0, q = 0;
  seg_load(0, 0, nx);
  while (k < N) {
    wave_lds_sync();  // the previous segment's reads of the LDS tile are done
#pragma unroll
    for (int u = 0; u < NV; ++u) {
      const int e = l + 64 * u;
      *reinterpret_cast<f4*>(&sx[e / (SEG / 4)][4 * (e % (SEG / 4))]) = nx[u];
    }
    wave_lds_sync();
    const int kc = k, qc = q;  // the segment in LDS
    if (++q * SEG >= a.n[k]) {
      ++k;
      q = 0;
    }
    if (k < N) seg_load(k, q, nx);  // the next segment, in flight during the contraction
    const int st = a.st[kc] + SEG * qc, nb = min(SEG, a.n[kc] - SEG * qc);
    sfor<0, N>([&](auto lc) {
      constexpr int lv = lc;
      if (lv != kc) return;
      const int en = a.st[lv] + a.n[lv];
#pragma unroll 2
      for (int cb = 0; cb < nb; cb += 16) {
        f4 xa[RT];
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
          xa[rt] = *reinterpret_cast<const f4*>(&sx[16 * rt + i][cb + 4 * g]);  // zero past the level's end
          ssq[lv][rt] = fmaf(xa[rt].x, xa[rt].x,
                             fmaf(xa[rt].y, xa[rt].y, fmaf(xa[rt].z, xa[rt].z, fmaf(xa[rt].w, xa[rt].w, ssq[lv][rt]))));
        }
        const int kk = st + cb + 4 * g;
#pragma unroll
        for (int h = 0; h < NH; ++h) {
          const int hrow = 16 * h + i;
          const bool hok = hrow < a.hidden;
          const f4 wb = load4(a.weight + (size_t)(hok ? hrow : 0) * a.D, kk, en, hok);
#pragma unroll
          for (int rt = 0; rt < RT; ++rt) {
            acc[lv][h][rt] = mfma(xa[rt].x, wb.x, acc[lv][h][rt]);
            acc[lv][h][rt] = mfma(xa[rt].y, wb.y, acc[lv][h][rt]);
            acc[lv][h][rt] = mfma(xa[rt].z, wb.z, acc[lv][h][rt]);
            acc[lv][h][rt] = mfma(xa[rt].w, wb.w, acc[lv][h][rt]);
          }
        }
      }
    });
  }
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    // per-row factors: lanes (i, g) hold partial sums of squares of row i; every lane of row i ends with the sum
    float fr[N];
    const int gi = row0 + 16 * rt + i;
    const bool vi = gi < M;
    sfor<0, N>([&](auto kc) {
      constexpr int kx = kc;
      float v = ssq[kx][rt];
      v = lanes::add_xor32(lanes::add_xor16(v));
      const int t = vi ? gi % a.R : 0;
      const int K = kx + 1;
      float c = 1.0f;
      if (a.prescale) {  // 1 / C(max(t + 1 + prepend, K), K), K <= 3: the exact product
        const double tl = fmax((double)(t + 1 + a.prepend), (double)K);
        c = (float)(K == 1 ? 1.0 / tl : (K == 2 ? 2.0 / (tl * (tl - 1.0)) : 6.0 / (tl * (tl - 1.0) * (tl - 2.0))));
      }
      float f, beta = 0.0f, dfdg;
      if (a.variant == EWS_GRADED_LIVE_RMS) {
        const float gk = a.gains[kx];
        const float ms = v / (float)a.n[kx];
        const float rho = ms > 0.0f ? sqrtf(ms) : 0.0f;
        const float den = fmaf(c, rho, a.eps[kx]);
        dfdg = c / den;
        f = gk * dfdg;
        if (rho > 0.0f) beta = gk * c * c / (den * den * (float)a.n[kx] * rho);
      } else if (a.variant == EWS_GRADED_STATIC_GAIN) {
        dfdg = c;
        f = a.gains[kx] * c;
      } else {
        const float lam = a.gains[0];
        const float lk1 = powf(lam, (float)(K - 1));
        dfdg = (float)K * lk1 * c;
        f = lk1 * lam * c;
      }
      fr[kx] = f;
      if (vi && g == kx) {  // one lane per (row, level) writes the residual's factors
        float* fp = a.F + ((size_t)gi * N + kx) * 3;
        fp[0] = f;
        fp[1] = beta;
        fp[2] = dfdg;
      }
    });
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int row = 4 * g + r, grow = row0 + 16 * rt + row;
      float fk[N];
#pragma unroll
      for (int kx = 0; kx < N; ++kx) fk[kx] = __shfl(fr[kx], row, 64);  // lane `row` holds row `row`'s factors
#pragma unroll
      for (int h = 0; h < NH; ++h) {
        const int col = 16 * h + i;
        if (grow < M && col < a.hidden) {
          float v = a.bias[col];
#pragma unroll
          for (int kx = 0; kx < N; ++kx) {
            const f4 qv = acc[kx][h][rt];
            const float pv = r == 0 ? qv.x : (r == 1 ? qv.y : (r == 2 ? qv.z : qv.w));
            v = fmaf(fk[kx], pv, v);
            a.P[((size_t)grow * N + kx) * a.hidden + col] = pv;
          }
          a.out[out_row(a, grow) * a.hidden + col] = v;
        }
      }
    }
  }
}

// the leading zero rows of the levels map to the bias alone
__global__ void k_mix_bias_rows(MArgs a) {
  const int b = blockIdx.x;
  for (int col = threadIdx.x; col < a.hidden; col += blockDim.x)
    a.out[(size_t)b * (a.R + 1) * a.hidden + col] = a.bias[col];
}

// Backward: a workgroup = 4 wavefronts x RT tiles of 16 rows (launched with RT = 1); every column block of every
// level. The RT row tiles of a wavefront would share each load of c_down's column block.
template <int N, int RT>
__global__ __launch_bounds__(256) void k_mix_bwd(MArgs a) {
  __shared__ float s_c[4][RT][3][2][16];
  const int w = threadIdx.x >> 6, l = threadIdx.x & 63, i = l & 15, g = l >> 4;
  const int M = a.B * a.R;
  const int row0 = (blockIdx.x * 4 + w) * 16 * RT;
  const float* drp[RT];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    const int gr = row0 + 16 * rt + i;
    const bool valid = gr < M;
    drp[rt] = a.gout + (valid ? out_row(a, gr) : 0) * a.hidden;
    // dot of each level's products with the row's cotangent (the four lanes of a row split the hidden columns)
    sfor<0, N>([&](auto kc) {
      constexpr int k = kc;
      float dot = 0.0f;
      if (valid) {
        const float* pp = a.P + ((size_t)gr * N + k) * a.hidden;
        for (int h = g; h < a.hidden; h += 4) dot = fmaf(pp[h], drp[rt][h], dot);
      }
      dot = lanes::add_xor32(lanes::add_xor16(dot));
      if (g == 0) {
        float f = 0.0f, bd = 0.0f;
        if (valid) {
          const float* fp = a.F + ((size_t)gr * N + k) * 3;
          f = fp[0];
          bd = fp[1] * dot;
          a.dots[(size_t)gr * N + k] = dot;
        }
        s_c[w][rt][k][0][i] = f;
        s_c[w][rt][k][1][i] = bd;
      }
    });
    if (a.lvl0 && valid && g == 0) a.grows[(size_t)gr * a.W] = 0.0f;
  }
  __syncthreads();
  sfor<0, N>([&](auto kc) {
    constexpr int k = kc;
    const int st = a.st[k], en = st + a.n[k];
    for (int c0 = st; c0 < en; c0 += 16) {
      const int col = c0 + i;  // this lane's column of the B operand and of the result
      const bool cok = col < en;
      f4 acc[RT];
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) acc[rt] = f4{0.0f, 0.0f, 0.0f, 0.0f};
      for (int h0 = 0; h0 < a.hidden; h0 += 16) {
        const int hh = h0 + 4 * g;
        float wv[4];
#pragma unroll
        for (int s = 0; s < 4; ++s)
          wv[s] = (cok && hh + s < a.hidden) ? a.weight[(size_t)(hh + s) * a.D + col] : 0.0f;
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
          const f4 da = load4(drp[rt], hh, a.hidden, row0 + 16 * rt + i < M);
          acc[rt] = mfma(da.x, wv[0], acc[rt]);
          acc[rt] = mfma(da.y, wv[1], acc[rt]);
          acc[rt] = mfma(da.z, wv[2], acc[rt]);
          acc[rt] = mfma(da.w, wv[3], acc[rt]);
        }
      }
      if (cok) {
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int row = 4 * g + r, grow = row0 + 16 * rt + row;
            if (grow < M) {
              const size_t e = (size_t)grow * a.W + a.lvl0 + col;
              const float dy = r == 0 ? acc[rt].x : (r == 1 ? acc[rt].y : (r == 2 ? acc[rt].z : acc[rt].w));
              a.grows[e] = fmaf(s_c[w][rt][k][0][row], dy, -s_c[w][rt][k][1][row] * a.rows[e]);
            }
          }
        }
      }
    }
  });
}

// Backward in two kernels, for c_down up to 128 wide. First, per row, the dot of each level's products with the
// row's cotangent (row_dots) and the zero level-0 cotangent. Then the columns: a wavefront owns two 16-column
// tiles, keeps their c_down blocks in registers (W[h][c], h < hidden) and walks a chunk of 16-row tiles:
// dy = dr W (MFMA, contraction over the hidden columns), dx = f dy - beta dot x with each lane's own level (a
// tile may straddle two levels). Each row element is read once; the chunk's output cotangents (hidden floats per
// row) are shared through L2 by the column workgroups of the chunk, which are consecutive in the grid.
constexpr int BW_HB = 8;    // hidden blocks of 16 held in registers: hidden <= 128 (4 up to 64)
constexpr int BW_RC = 32;   // row tiles per workgroup chunk

// a lane per row and level: the dot of the level's products with the row's cotangent, in 16-byte runs
__global__ __launch_bounds__(256) void k_mix_bwd_dots(MArgs a) {
  const int M = a.B * a.R;
  const int q = blockIdx.x * blockDim.x + threadIdx.x;
  if (q >= M * a.N) return;
  const int gr = q / a.N, k = q - gr * a.N;
  const float* drp = a.gout + out_row(a, gr) * a.hidden;
  const float* pp = a.P + ((size_t)gr * a.N + k) * a.hidden;
  float dot = 0.0f;
  for (int h = 0; h < a.hidden; h += 4) {
    const f4 p = load4(pp, h, a.hidden, true), r = load4(drp, h, a.hidden, true);
    dot = fmaf(p.x, r.x, fmaf(p.y, r.y, fmaf(p.z, r.z, fmaf(p.w, r.w, dot))));
  }
  a.dots[(size_t)gr * a.N + k] = dot;
  if (a.lvl0 && k == 0) a.grows[(size_t)gr * a.W] = 0.0f;
}

// XCD-aware order: the hardware deals consecutive workgroups round-robin to the 8 XCDs (each with its own L2);
// renumbering by (id mod 8, id / 8) gives each XCD a contiguous run of logical workgroups, so the column workgroups
// of one row chunk share an L2 (their output-cotangent rows and the two halves of every row line)
__device__ __forceinline__ int xcd_logical(int hw, int total) {
  const int per = total >> 3;  // total is a multiple of 8
  return (hw & 7) * per + (hw >> 3);
}

// Row access: each wavefront moves its 16 x 32 block of a row tile between memory and a private LDS tile with
// 16-byte row-segment loads and stores (8 lanes per row: one 128-byte run), and reads it there in the MFMA layout;
// the next tile's block is loaded into registers while the current one is worked on. A wavefront's LDS tile is its
// own, so the hand-offs need no workgroup barrier (a wavefront's LDS operations complete in program order).
// DW: the same pass also accumulates c_down's weight gradient over the chunk, dW[h][c] = sum_rows dr[h] f x[c]
// (MFMA with the rows as the contraction: A = the output cotangent of rows 4 g + s at hidden column 16 hb + i,
// B = f x of the lane's own row elements), and writes the chunk's partial; k_mix_dw_reduce sums the partials.
constexpr int BW_XP = 36;  // LDS row pitch of a wavefront's 16 x 32 tile (16-byte rows, 2-way bank spread)


__device__ __forceinline__ f4 ld_row4(const float* p, int c, int nc, bool ok) {
  // p[c .. c+3] of a row segment whose valid columns end at nc (dword-aligned; unaligned 16-byte loads are fine)
  if (!ok) return f4{0.0f, 0.0f, 0.0f, 0.0f};
  if (c + 3 < nc) {
    const f4u v = *reinterpret_cast<const f4u*>(p + c);
    return f4{v.x, v.y, v.z, v.w};
  }
  return f4{c < nc ? p[c] : 0.0f, c + 1 < nc ? p[c + 1] : 0.0f, c + 2 < nc ? p[c + 2] : 0.0f,
            c + 3 < nc ? p[c + 3] : 0.0f};
}

template <int HB, bool DW>
__global__ __launch_bounds__(256) void k_mix_bwd_cols(MArgs a, int ncolwg, int nchunks) {
  const int w = threadIdx.x >> 6, l = threadIdx.x & 63, i = l & 15, g = l >> 4;
  const int M = a.B * a.R;
  const int total = gridDim.x;
  const int lid = xcd_logical(blockIdx.x, total);
  const int cwg = lid % ncolwg, chunk = lid / ncolwg;
  if (chunk >= nchunks) return;  // padding of the grid to a multiple of 8 (uniform over the workgroup)
  // two 16-column tiles per wavefront: a row's 32 columns of one wavefront are one 128-byte run
  const int cbase = (cwg * 4 + w) * 32;
  int col[2], lev[2];
  bool cok[2];
#pragma unroll
  for (int ct = 0; ct < 2; ++ct) {
    col[ct] = cbase + 16 * ct + i;
    cok[ct] = col[ct] < a.D;
    lev[ct] = 0;
    for (int k = 1; k < a.N; ++k)
      if (col[ct] >= a.st[k]) lev[ct] = k;
  }
  const int nhb = (a.hidden + 15) / 16;
  float wr[2][HB][4];  // c_down blocks of the two tiles: W[16 hb + 4 g + s][col]
#pragma unroll
  for (int ct = 0; ct < 2; ++ct)
#pragma unroll
    for (int hb = 0; hb < HB; ++hb)
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const int h = 16 * hb + 4 * g + s;
        wr[ct][hb][s] = (hb < nhb && cok[ct] && h < a.hidden) ? a.weight[(size_t)h * a.D + col[ct]] : 0.0f;
      }
  // per-row factors of each level (scale f, correction beta * dot) of the chunk's rows, staged once
  __shared__ float s_fb[BW_RC * 16][3][2];
  __shared__ __align__(16) float s_x[4][16][BW_XP];  // each wavefront's row tile: x, then its cotangent
  __shared__ __align__(16) float s_gt[DW ? 4 : 1][16][DW ? 16 * HB + 4 : 1];  // DW: the tile's output cotangents
  const int t0 = chunk * BW_RC, tiles = (M + 15) / 16, t1 = min(t0 + BW_RC, tiles);
  for (int q = threadIdx.x; q < BW_RC * 16 * a.N; q += blockDim.x) {
    const int r = q / a.N, k = q - r * a.N, grow = t0 * 16 + r;
    float f = 0.0f, bd = 0.0f;
    if (grow < M) {
      const float* fp = a.F + ((size_t)grow * a.N + k) * 3;
      f = fp[0];
      bd = fp[1] * a.dots[(size_t)grow * a.N + k];
    }
    s_fb[r][k][0] = f;
    s_fb[r][k][1] = bd;
  }
  __syncthreads();
  float(*sx)[BW_XP] = s_x[w];
  // row-segment lanes: rows l / 8 and 8 + l / 8 of the tile, columns 4 (l % 8) .. + 3 of the wavefront's block
  const int sr = l >> 3, sc = 4 * (l & 7);
  const int nc = a.D - cbase;  // valid columns of the block (<= 0: none)
  f4 xn[2];
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    const int grow = t0 * 16 + sr + 8 * q;
    xn[q] = ld_row4(a.rows + (size_t)(grow < M ? grow : 0) * a.W + a.lvl0 + cbase, sc, nc, grow < M && nc > 0);
  }
  f4 dacc[DW ? 2 : 1][DW ? HB : 1];
#pragma unroll
  for (int ct = 0; ct < (DW ? 2 : 1); ++ct)
#pragma unroll
    for (int hb = 0; hb < (DW ? HB : 1); ++hb) dacc[ct][hb] = f4{0.0f, 0.0f, 0.0f, 0.0f};
  for (int tt = t0; tt < t1; ++tt) {
    const int row0 = tt * 16, lr0 = row0 - t0 * 16;
    wave_lds_sync();  // the previous tile's reads of the LDS tile are done
#pragma unroll
    for (int q = 0; q < 2; ++q) *reinterpret_cast<f4*>(&sx[sr + 8 * q][sc]) = xn[q];
    wave_lds_sync();
    if (tt + 1 < t1) {  // the next tile's block, in flight while this one is worked on
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        const int grow = row0 + 16 + sr + 8 * q;
        xn[q] = ld_row4(a.rows + (size_t)(grow < M ? grow : 0) * a.W + a.lvl0 + cbase, sc, nc, grow < M && nc > 0);
      }
    }
    const int ga = row0 + i;  // A-operand row of this lane
    const float* drp = a.gout + (ga < M ? out_row(a, ga) : 0) * a.hidden;
    f4 acc[2] = {f4{0.0f, 0.0f, 0.0f, 0.0f}, f4{0.0f, 0.0f, 0.0f, 0.0f}};
#pragma unroll
    for (int hb = 0; hb < HB; ++hb) {
      if (hb < nhb) {
        const f4 da = load4(drp, 16 * hb + 4 * g, a.hidden, ga < M);
        if constexpr (DW) *reinterpret_cast<f4*>(&s_gt[w][i][16 * hb + 4 * g]) = da;
#pragma unroll
        for (int ct = 0; ct < 2; ++ct) {
          acc[ct] = mfma(da.x, wr[ct][hb][0], acc[ct]);
          acc[ct] = mfma(da.y, wr[ct][hb][1], acc[ct]);
          acc[ct] = mfma(da.z, wr[ct][hb][2], acc[ct]);
          acc[ct] = mfma(da.w, wr[ct][hb][3], acc[ct]);
        }
      }
    }
    float fx[2][4];  // f x of the lane's row elements: rows 4 g + r of its two columns (zero past the rows)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int row = 4 * g + r;
#pragma unroll
      for (int ct = 0; ct < 2; ++ct) {
        float* px = &sx[row][16 * ct + i];
        const float x = *px;
        const float f = s_fb[lr0 + row][lev[ct]][0];
        const float dy = r == 0 ? acc[ct].x : (r == 1 ? acc[ct].y : (r == 2 ? acc[ct].z : acc[ct].w));
        fx[ct][r] = f * x;
        *px = fmaf(f, dy, -s_fb[lr0 + row][lev[ct]][1] * x);
      }
    }
    wave_lds_sync();
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const int grow = row0 + sr + 8 * q;
      if (grow < M && nc > 0) {
        const f4 v = *reinterpret_cast<const f4*>(&sx[sr + 8 * q][sc]);
        float* op = a.grows + (size_t)grow * a.W + a.lvl0 + cbase;
        if (sc + 3 < nc) {
          *reinterpret_cast<f4u*>(op + sc) = f4u{v.x, v.y, v.z, v.w};
        } else {
          if (sc < nc) op[sc] = v.x;
          if (sc + 1 < nc) op[sc + 1] = v.y;
          if (sc + 2 < nc) op[sc + 2] = v.z;
        }
      }
    }
    if constexpr (DW) {  // A: the cotangent of rows 4 g + s at hidden column 16 hb + i; B: f x
#pragma unroll
      for (int hb = 0; hb < HB; ++hb) {
        if (hb < nhb) {  // uniform
#pragma unroll
          for (int s = 0; s < 4; ++s) {
            const float gt = s_gt[w][4 * g + s][16 * hb + i];  // zero past the rows and the hidden columns
#pragma unroll
            for (int ct = 0; ct < 2; ++ct) dacc[ct][hb] = mfma(gt, fx[ct][s], dacc[ct][hb]);
          }
        }
      }
    }
  }
  if constexpr (DW) {  // lane: dW rows 16 hb + 4 g + r of its columns
#pragma unroll
    for (int ct = 0; ct < 2; ++ct) {
      if (!cok[ct]) continue;
#pragma unroll
      for (int hb = 0; hb < HB; ++hb) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int h = 16 * hb + 4 * g + r;
          if (hb < nhb && h < a.hidden) {
            const float v = r == 0 ? dacc[ct][hb].x : (r == 1 ? dacc[ct][hb].y : (r == 2 ? dacc[ct][hb].z : dacc[ct][hb].w));
            a.dwpart[((size_t)chunk * a.hidden + h) * a.D + col[ct]] = v;
          }
        }
      }
    }
  }
}

// c_down's weight gradient: the chunks' partials summed in float64 in a fixed order (deterministic). A
// workgroup owns 64 entries; wavefront w sums the w-th sixteenth of the chunks, then the sixteen sums are added in
// order.
constexpr int DW_RW = 16;  // wavefronts per reduction workgroup
__global__ __launch_bounds__(64 * DW_RW) void k_mix_dw_reduce(MArgs a, int nchunks, float* gw) {
  __shared__ double s_part[DW_RW][64];
  const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
  const size_t HD = (size_t)a.hidden * a.D;
  const size_t e = (size_t)blockIdx.x * 64 + l;
  const int per = (nchunks + DW_RW - 1) / DW_RW, c0 = w * per, c1 = min(nchunks, c0 + per);
  double s = 0.0;
  if (e < HD) {
#pragma unroll 4
    for (int c = c0; c < c1; ++c) s += (double)a.dwpart[(size_t)c * HD + e];
  }
  s_part[w][l] = s;
  __syncthreads();
  if (w == 0 && e < HD) {
    double t = 0.0;
    for (int k = 0; k < DW_RW; ++k) t += s_part[k][l];
    gw[e] = (float)t;
  }
}

}  // namespace mixer
}  // namespace ews

// ================================================================================================= C ABI
namespace {

using namespace ews::mixer;

size_t al256m(size_t x) { return (x + 255) & ~(size_t)255; }

struct MPlan {
  MArgs a;
  size_t P, F, total;
};

int mixer_plan(const ews_mixer_desc* s, MPlan& p) {
  if (!s) return EWS_ERR_NULL;
  if (s->depth < 1 || s->depth > 3) return EWS_ERR_DEPTH;
  if (s->variant < 0 || s->variant > 2) return EWS_ERR_OPTION;
  if (s->batch < 1 || s->rows < 1 || s->dim < 1 || s->dim > 64 || s->hidden < 1) return EWS_ERR_SHAPE;
  if (s->depth == 3 && s->dim > 16) return EWS_ERR_SHAPE;
  MArgs& a = p.a;
  a = MArgs{};
  a.B = s->batch;
  a.R = s->rows;
  a.d = s->dim;
  a.N = s->depth;
  a.lvl0 = s->level0 ? 1 : 0;
  a.hidden = s->hidden;
  a.variant = s->variant;
  a.prepend = s->prepend ? 1 : 0;
  a.prescale = s->prescale ? 1 : 0;
  int D = 0;
  for (int k = 0, m = 1; k < a.N; ++k) {
    m *= a.d;
    a.st[k] = D;
    a.n[k] = m;
    a.eps[k] = s->eps[k];
    D += m;
  }
  a.D = D;
  a.W = D + a.lvl0;
  const size_t M = (size_t)a.B * a.R;
  size_t off = 0;
  p.P = off;
  off += al256m(M * a.N * a.hidden * 4);
  p.F = off;
  off += al256m(M * a.N * 3 * 4);
  p.total = off;
  return EWS_OK;
}

#define MIX_CHECK()                                            \
  do {                                                         \
    if (hipGetLastError() != hipSuccess) return EWS_ERR_LAUNCH; \
  } while (0)

}  // namespace

extern "C" {

size_t ews_mixer_residual_bytes(const ews_mixer_desc* desc) {
  MPlan p;
  if (mixer_plan(desc, p) != EWS_OK) return 0;
  return p.total;
}

int ews_mixer_forward(const ews_mixer_desc* desc, const float* rows, const float* weight, const float* bias,
                      const float* gains, float* out, void* residual, ews_stream_t stream) {
  MPlan p;
  const int rc = mixer_plan(desc, p);
  if (rc != EWS_OK) return rc;
  if (!rows || !weight || !bias || !gains || !out || !residual) return EWS_ERR_NULL;
  MArgs a = p.a;
  a.rows = rows;
  a.weight = weight;
  a.bias = bias;
  a.gains = gains;
  a.out = out;
  a.P = (float*)((char*)residual + p.P);
  a.F = (float*)((char*)residual + p.F);
  hipStream_t st = (hipStream_t)stream;
  const int M = a.B * a.R;
  // hidden tiles per pass: two when c_down is at most 32 wide, else four; two row tiles per wavefront share each
  // c_down load once there are rows enough (depths 1-2: the depth-3 accumulators would cost occupancy)
  const int NH = a.hidden <= 32 ? 2 : 4;
  const int RT = (M >= 256 * 1024 && a.N <= 2) ? 2 : 1;
  const dim3 grid((M + 64 * RT - 1) / (64 * RT), (a.hidden + 16 * NH - 1) / (16 * NH)), blk(256);
  if (a.hidden <= 64) {  // streamed rows, every hidden column in one wavefront
    // one row tile per wavefront: two (half the c_down loads, 64-entry segments, fewer waves per SIMD) measured
    // 0.433 ms against 0.418 ms on the c5 epilogue (depth 2, 24 columns, 399K rows)
#define MIX_FWD_S(NN, H) hipLaunchKernelGGL((k_mix_fwd_s<NN, H, 1>), dim3((M + 63) / 64), blk, 0, st, a)
    if (a.N == 1) {
      if (NH == 2) MIX_FWD_S(1, 2);
      else MIX_FWD_S(1, 4);
    } else if (a.N == 2) {
      if (NH == 2) MIX_FWD_S(2, 2);
      else MIX_FWD_S(2, 4);
    } else {
      if (NH == 2) MIX_FWD_S(3, 2);
      else MIX_FWD_S(3, 4);
    }
#undef MIX_FWD_S
    MIX_CHECK();
    if (a.prepend) {
      hipLaunchKernelGGL(k_mix_bias_rows, dim3(a.B), dim3(64), 0, st, a);
      MIX_CHECK();
    }
    return EWS_OK;
  }
#define MIX_FWD(NN, H, T) hipLaunchKernelGGL((k_mix_fwd<NN, H, T>), grid, blk, 0, st, a)
  if (a.N == 1) {
    if (NH == 2) { if (RT == 2) MIX_FWD(1, 2, 2); else MIX_FWD(1, 2, 1); }
    else { if (RT == 2) MIX_FWD(1, 4, 2); else MIX_FWD(1, 4, 1); }
  } else if (a.N == 2) {
    if (NH == 2) { if (RT == 2) MIX_FWD(2, 2, 2); else MIX_FWD(2, 2, 1); }
    else { if (RT == 2) MIX_FWD(2, 4, 2); else MIX_FWD(2, 4, 1); }
  } else {
    if (NH == 2) MIX_FWD(3, 2, 1);
    else MIX_FWD(3, 4, 1);
  }
#undef MIX_FWD
  MIX_CHECK();
  if (a.prepend) {
    hipLaunchKernelGGL(k_mix_bias_rows, dim3(a.B), dim3(64), 0, st, a);
    MIX_CHECK();
  }
  return EWS_OK;
}

size_t ews_mixer_backward_workspace_bytes(const ews_mixer_desc* desc) {
  MPlan p;
  if (mixer_plan(desc, p) != EWS_OK || p.a.hidden > 16 * BW_HB) return 0;
  const int tiles = (p.a.B * p.a.R + 15) / 16, nchunks = (tiles + BW_RC - 1) / BW_RC;
  return al256m((size_t)nchunks * p.a.hidden * p.a.D * 4);
}

int ews_mixer_backward_weight(const ews_mixer_desc* desc, const float* rows, const float* weight,
                              const void* residual, const float* grad_out, float* grad_rows, float* row_dots,
                              float* grad_weight, void* workspace, ews_stream_t stream) {
  MPlan p;
  const int rc = mixer_plan(desc, p);
  if (rc != EWS_OK) return rc;
  if (p.a.hidden > 16 * BW_HB) return EWS_ERR_SHAPE;
  if (!rows || !weight || !residual || !grad_out || !grad_rows || !row_dots || !grad_weight || !workspace)
    return EWS_ERR_NULL;
  MArgs a = p.a;
  a.rows = rows;
  a.weight = weight;
  a.P = (float*)((char*)residual + p.P);
  a.F = (float*)((char*)residual + p.F);
  a.gout = grad_out;
  a.grows = grad_rows;
  a.dots = row_dots;
  a.dwpart = (float*)workspace;
  hipStream_t st = (hipStream_t)stream;
  const int M = a.B * a.R;
  const dim3 blk(256);
  hipLaunchKernelGGL(k_mix_bwd_dots, dim3((M * a.N + 255) / 256), blk, 0, st, a);
  MIX_CHECK();
  const int tiles = (M + 15) / 16;
  const int ncolwg = (a.D + 127) / 128, nchunks = (tiles + BW_RC - 1) / BW_RC;
  const int total = (ncolwg * nchunks + 7) / 8 * 8;
  if (a.hidden <= 32) hipLaunchKernelGGL((k_mix_bwd_cols<2, true>), dim3(total), blk, 0, st, a, ncolwg, nchunks);
  else if (a.hidden <= 64) hipLaunchKernelGGL((k_mix_bwd_cols<4, true>), dim3(total), blk, 0, st, a, ncolwg, nchunks);
  else hipLaunchKernelGGL((k_mix_bwd_cols<BW_HB, true>), dim3(total), blk, 0, st, a, ncolwg, nchunks);
  MIX_CHECK();
  const size_t HD = (size_t)a.hidden * a.D;
  hipLaunchKernelGGL(k_mix_dw_reduce, dim3((unsigned)((HD + 63) / 64)), dim3(64 * DW_RW), 0, st, a, nchunks,
                     grad_weight);
  MIX_CHECK();
  return EWS_OK;
}

int ews_mixer_backward(const ews_mixer_desc* desc, const float* rows, const float* weight, const void* residual,
                       const float* grad_out, float* grad_rows, float* row_dots, ews_stream_t stream) {
  MPlan p;
  const int rc = mixer_plan(desc, p);
  if (rc != EWS_OK) return rc;
  if (!rows || !weight || !residual || !grad_out || !grad_rows || !row_dots) return EWS_ERR_NULL;
  MArgs a = p.a;
  a.rows = rows;
  a.weight = weight;
  a.P = (float*)((char*)residual + p.P);
  a.F = (float*)((char*)residual + p.F);
  a.gout = grad_out;
  a.grows = grad_rows;
  a.dots = row_dots;
  hipStream_t st = (hipStream_t)stream;
  const int M = a.B * a.R;
  const dim3 blk(256);
  if (a.hidden <= 16 * BW_HB) {
    // rows' dots, then column tiles over chunks of row tiles (column workgroups of a chunk consecutive)
    hipLaunchKernelGGL(k_mix_bwd_dots, dim3((M * a.N + 255) / 256), blk, 0, st, a);
    MIX_CHECK();
    const int tiles = (M + 15) / 16;
    const int ncolwg = (a.D + 127) / 128, nchunks = (tiles + BW_RC - 1) / BW_RC;
    const int total = (ncolwg * nchunks + 7) / 8 * 8;  // the XCD renumbering needs a multiple of 8
    if (a.hidden <= 64) hipLaunchKernelGGL((k_mix_bwd_cols<4, false>), dim3(total), blk, 0, st, a, ncolwg, nchunks);
    else hipLaunchKernelGGL((k_mix_bwd_cols<BW_HB, false>), dim3(total), blk, 0, st, a, ncolwg, nchunks);
  } else {
    // wider c_down: a wavefront per 16 rows, every column block (c_down re-read per row tile)
    const dim3 grid((M + 63) / 64);
    if (a.N == 1) hipLaunchKernelGGL((k_mix_bwd<1, 1>), grid, blk, 0, st, a);
    else if (a.N == 2) hipLaunchKernelGGL((k_mix_bwd<2, 1>), grid, blk, 0, st, a);
    else hipLaunchKernelGGL((k_mix_bwd<3, 1>), grid, blk, 0, st, a);
  }
  MIX_CHECK();
  return EWS_OK;
}

}  // extern "C"
