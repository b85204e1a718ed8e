// Row-wise and element-wise kernels of the eSCN-MD path: the gate activation (m-primed for the
// SO(2) block, natural order for the spectral feed-forward), the radial MLP's fused
// LayerNorm+SiLU forward/backward, the equivariant RMS norm over SH coefficients and small
// deterministic reductions.
#include "common.h"

typedef float floatx4 __attribute__((ext_vector_type(4)));

namespace {

struct GateIdx {
  int v[8];  // gate row per vector coefficient 1..8
};

// GateActivation (activation.py:29-70, spectral.py:129-144):
//   y[r, 0, h] = silu(x[r, 0, h]);  y[r, c, h] = x[r, c, h] * sigmoid(gating[r, idx[c-1] * H + h])
// x and gating rows have strides ldx / ldg (they may be column blocks of one GEMM output row).
__global__ __launch_bounds__(256) void k_gate_fwd(const float* __restrict__ x,
                                                  const float* __restrict__ gating,
                                                  float* __restrict__ y, int64_t R, int H, int L,
                                                  int64_t ldx, int64_t ldg, GateIdx idx) {
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= R * H) return;
  const int64_t r = gid / H;
  const int h = (int)(gid % H);
  const float* xr = x + r * ldx;
  float* yr = y + r * 9 * H;
  float sg[8];
  for (int t = 0; t < L; ++t) sg[t] = tta_sigmoid_acc(gating[r * ldg + t * H + h]);
  yr[h] = tta_silu(xr[h]);
#pragma unroll
  for (int c = 1; c < 9; ++c) yr[c * H + h] = xr[c * H + h] * sg[idx.v[c - 1]];
}

// Backward (forces.py:104-130): g_x and g_gating = sigmoid'(gating) * sum_c g_y[c] x[c].
// g_x rows share x's stride ldx, g_gating rows share gating's stride ldg.
__global__ __launch_bounds__(256) void k_gate_bwd(const float* __restrict__ g_y,
                                                  const float* __restrict__ x,
                                                  const float* __restrict__ gating,
                                                  float* __restrict__ g_x,
                                                  float* __restrict__ g_gating, int64_t R, int H,
                                                  int L, int64_t ldx, int64_t ldg, GateIdx idx) {
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= R * H) return;
  const int64_t r = gid / H;
  const int h = (int)(gid % H);
  const float* xr = x + r * ldx;
  const float* gr = g_y + r * 9 * H;
  float* gx = g_x + r * ldx;
  float sg[8], acc[8];
  for (int t = 0; t < L; ++t) {
    sg[t] = tta_sigmoid_acc(gating[r * ldg + t * H + h]);
    acc[t] = 0.f;
  }
  // streaming stores for the [R, 9, H] adjoint (-7 % on the C3 step; the forward gate's output,
  // read at once by the next product, measured faster with ordinary stores)
  __builtin_nontemporal_store(gr[h] * tta_silu_grad(xr[h]), gx + h);
#pragma unroll
  for (int c = 1; c < 9; ++c) {
    const int t = idx.v[c - 1];
    const float g = gr[c * H + h];
    __builtin_nontemporal_store(g * sg[t], gx + c * H + h);
    acc[t] += g * xr[c * H + h];
  }
  for (int t = 0; t < L; ++t) g_gating[r * ldg + t * H + h] = acc[t] * (sg[t] * (1.f - sg[t]));
}

// The gating adjoint of a gate whose forward ran in the producing GEMM's epilogue and whose input
// adjoint g_x (g_x[c] = g_y[c] s[t_c], coefficient 0 aside) the adjoint GEMM's epilogue wrote:
// with y[c] = x[c] s[t] (the gated rows kept from the forward) and s = sigmoid(gating),
//   g_gating[t] = sigmoid'(gating[t]) sum_c g_y[c] x[c] = ((1 - s[t]) / s[t]) sum_c g_x[c] y[c]
// over the coefficients c > 0 of degree index t (forces.py:104-130); an s that underflowed to 0
// gives 0 (its true value is below 2^-126 times the sum).  y contiguous [R, 9, H]; g_x, sig and
// g_gating have their own row strides.
__global__ __launch_bounds__(256) void k_gate_gating_bwd(
    const float* __restrict__ g_x, const float* __restrict__ y, const float* __restrict__ sig,
    float* __restrict__ g_gating, int64_t R, int H, int L, int64_t ldgx, int64_t ldg,
    int64_t ldgg, GateIdx idx) {
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= R * H) return;
  const int64_t r = gid / H;
  const int h = (int)(gid % H);
  const float* yr = y + r * 9 * H;
  const float* gr = g_x + r * ldgx;
  float acc[8];
  for (int t = 0; t < L; ++t) acc[t] = 0.f;
#pragma unroll
  for (int c = 1; c < 9; ++c) acc[idx.v[c - 1]] += gr[c * H + h] * yr[c * H + h];
  for (int t = 0; t < L; ++t) {
    const float sg = sig[r * ldg + t * H + h];
    g_gating[r * ldgg + t * H + h] = sg > 0.f ? acc[t] * ((1.f - sg) / sg) : 0.f;
  }
}

// ------------------------------------------------------------------ LayerNorm + SiLU (radial MLP)
// G lanes per row (64; 16 for rows of 65 to 128, so that a wavefront holds four rows and a lane
// two float4 groups of its row in flight; 32 below); the row stays in registers (element NPL
// lane + k in slot k,
// NPL slots) so that each operand crosses HBM once.  The per-lane partial sums run over k in
// order.  The float4 path (VEC) and the element-wise path hold the same columns in the same
// slots and are compiled without fused multiply-adds, so both round every operation alike
// whichever path the forward and the backward take (the backward's recomputed LayerNorm output
// equals the forward's bit for bit).  A row index past R (the odd tail of a two-row wavefront) reads row R - 1 and stores
// nothing, so every lane of the wave takes part in the butterflies.  Forward (so2.py:101-115 /
// geometry.py:161-168):
//   nrm = (a - mean) * rstd * gamma + beta,  s = silu(nrm)
// a and nrm rows have stride lda, s rows stride lds.  `groups` independent LayerNorms per row
// (the radial MLPs of several blocks side by side): group k of a row is the n columns from k n,
// with gamma / beta [groups, n]; a row of a wavefront is one (row, group) pair.
template <int G, int NPL, bool VEC>
__global__ __launch_bounds__(256) void k_ln_silu_fwd(const float* __restrict__ a,
                                                     const float* __restrict__ gamma,
                                                     const float* __restrict__ beta,
                                                     float* __restrict__ nrm,
                                                     float* __restrict__ s, int64_t R, int n,
                                                     int groups, int64_t lda, int64_t lds,
                                                     float eps) {
  // no fused multiply-adds: the float4 and the element-wise paths (and the forward and the
  // backward's recomputation) then round every operation alike
#pragma clang fp contract(off)
  const int64_t RV = R * groups;
  const int64_t rw = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) / G;
  const int lane = threadIdx.x & (G - 1);
  if ((rw / (64 / G)) * (64 / G) >= RV) return;  // whole wavefront past the end
  const bool valid = rw < RV;
  const int64_t vr = valid ? rw : RV - 1;
  const int64_t row = vr / groups;
  const int co = (int)(vr - row * groups) * n;  // column offset of the group
  gamma += co;
  beta += co;
  const float* ar = a + row * lda + co;
  // element k of lane l: column NPL l + k; with VEC (n = 4 G, 16-byte aligned rows) all four
  // in one float4
  float v[NPL];
  if constexpr (VEC) {
    static_assert(NPL % 4 == 0, "float4 groups");
#pragma unroll
    for (int b = 0; b < NPL / 4; ++b) {
      const floatx4 x = *reinterpret_cast<const floatx4*>(ar + NPL * lane + 4 * b);
#pragma unroll
      for (int k = 0; k < 4; ++k) v[4 * b + k] = x[k];
    }
  }
  float sum = 0.f;
#pragma unroll
  for (int k = 0; k < NPL; ++k) {
    if constexpr (!VEC) {
      const int i = NPL * lane + k;
      v[k] = i < n ? ar[i] : 0.f;
    }
    sum += v[k];
  }
  const float mean = tta_group_sum(sum, G) / n;
  float sq = 0.f;
#pragma unroll
  for (int k = 0; k < NPL; ++k) {
    const float d = v[k] - mean;
    if (VEC || NPL * lane + k < n) sq += d * d;
  }
  const float var = tta_group_sum(sq, G) / n;
  const float rstd = 1.0f / sqrtf(var + eps);
  if (!valid) return;
  if constexpr (VEC) {
#pragma unroll
    for (int b = 0; b < NPL / 4; ++b) {
      const int c4 = NPL * lane + 4 * b;
      const floatx4 gm = *reinterpret_cast<const floatx4*>(gamma + c4);
      const floatx4 bt = *reinterpret_cast<const floatx4*>(beta + c4);
      floatx4 y, sv;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        y[k] = (v[4 * b + k] - mean) * rstd * gm[k] + bt[k];
        sv[k] = tta_silu(y[k]);
      }
      if (nrm) *reinterpret_cast<floatx4*>(nrm + row * lda + co + c4) = y;
      *reinterpret_cast<floatx4*>(s + row * lds + co + c4) = sv;
    }
    return;
  }
#pragma unroll
  for (int k = 0; k < NPL; ++k) {
    const int i = NPL * lane + k;
    if (i >= n) continue;
    const float y = (v[k] - mean) * rstd * gamma[i] + beta[i];
    if (nrm) nrm[row * lda + co + i] = y;
    s[row * lds + co + i] = tta_silu(y);
  }
}

// Backward of silu(layer_norm(a)) w.r.t. a (so2.py:117-143):
//   gy = g * silu'(nrm) * gamma;  xhat = (a - mean) * rstd;
//   g_a = rstd * (gy - mean(gy) - xhat * mean(gy * xhat))
// g rows stride ldg, a / nrm rows stride lda, g_a rows stride ldo.  Same lane layout as above.
// RECOMP: nrm is not read but recomputed from a, gamma and beta with the forward's operations
// (the same row statistics and the same expression, so the same values).
template <int G, int NPL, bool RECOMP, bool VEC>
__global__ __launch_bounds__(256) void k_ln_silu_bwd(const float* __restrict__ g,
                                                     const float* __restrict__ a,
                                                     const float* __restrict__ nrm,
                                                     const float* __restrict__ gamma,
                                                     const float* __restrict__ beta,
                                                     float* __restrict__ g_a, int64_t R, int n,
                                                     int groups, int64_t ldg, int64_t lda,
                                                     int64_t ldo, float eps) {
  // no fused multiply-adds: the float4 and the element-wise paths (and the forward and the
  // backward's recomputation) then round every operation alike
#pragma clang fp contract(off)
  const int64_t RV = R * groups;
  const int64_t rw = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) / G;
  const int lane = threadIdx.x & (G - 1);
  if ((rw / (64 / G)) * (64 / G) >= RV) return;
  const bool valid = rw < RV;
  const int64_t vr = valid ? rw : RV - 1;
  const int64_t row = vr / groups;
  const int co = (int)(vr - row * groups) * n;
  gamma += co;
  if (RECOMP) beta += co;
  const float* ar = a + row * lda + co;
  float av[NPL], gy[NPL];
  float sum = 0.f;
  // element layout as in k_ln_silu_fwd
  if constexpr (VEC) {
    static_assert(NPL % 4 == 0, "float4 groups");
#pragma unroll
    for (int b = 0; b < NPL / 4; ++b) {
      const int c4 = NPL * lane + 4 * b;
      const floatx4 x = *reinterpret_cast<const floatx4*>(ar + c4);
      const floatx4 gv = *reinterpret_cast<const floatx4*>(g + row * ldg + co + c4);
      floatx4 nv = {0.f, 0.f, 0.f, 0.f}, gm = {0.f, 0.f, 0.f, 0.f};
      if constexpr (!RECOMP) {
        nv = *reinterpret_cast<const floatx4*>(nrm + row * lda + co + c4);
        gm = *reinterpret_cast<const floatx4*>(gamma + c4);
      }
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        av[4 * b + k] = x[k];
        gy[4 * b + k] = RECOMP ? gv[k] : gv[k] * tta_silu_grad(nv[k]) * gm[k];
        sum += av[4 * b + k];
      }
    }
  } else {
#pragma unroll
    for (int k = 0; k < NPL; ++k) {
      const int i = NPL * lane + k;
      const bool in = i < n;
      av[k] = in ? ar[i] : 0.f;
      if (RECOMP)
        gy[k] = in ? g[row * ldg + co + i] : 0.f;
      else
        gy[k] =
            in ? g[row * ldg + co + i] * tta_silu_grad(nrm[row * lda + co + i]) * gamma[i] : 0.f;
      sum += av[k];
    }
  }
  const float mean = tta_group_sum(sum, G) / n;
  float sq = 0.f;
#pragma unroll
  for (int k = 0; k < NPL; ++k) {
    const float d = av[k] - mean;
    if (VEC || NPL * lane + k < n) sq += d * d;
  }
  const float var = tta_group_sum(sq, G) / n;
  const float rstd = 1.0f / sqrtf(var + eps);
  if (RECOMP) {
    if constexpr (VEC) {
#pragma unroll
      for (int b = 0; b < NPL / 4; ++b) {
        const int c4 = NPL * lane + 4 * b;
        const floatx4 gm = *reinterpret_cast<const floatx4*>(gamma + c4);
        const floatx4 bt = *reinterpret_cast<const floatx4*>(beta + c4);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const float y = (av[4 * b + k] - mean) * rstd * gm[k] + bt[k];
          gy[4 * b + k] = gy[4 * b + k] * tta_silu_grad(y) * gm[k];
        }
      }
    } else {
#pragma unroll
      for (int k = 0; k < NPL; ++k) {
        const int i = NPL * lane + k;
        if (i >= n) continue;
        const float y = (av[k] - mean) * rstd * gamma[i] + beta[i];
        gy[k] = gy[k] * tta_silu_grad(y) * gamma[i];
      }
    }
  }
  float m1 = 0.f, m2 = 0.f;
#pragma unroll
  for (int k = 0; k < NPL; ++k) {
    m1 += gy[k];
    m2 += gy[k] * ((av[k] - mean) * rstd);
  }
  m1 = tta_group_sum(m1, G) / n;
  m2 = tta_group_sum(m2, G) / n;
  if (!valid) return;
  if constexpr (VEC) {
#pragma unroll
    for (int b = 0; b < NPL / 4; ++b) {
      floatx4 o;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const float xh = (av[4 * b + k] - mean) * rstd;
        o[k] = rstd * (gy[4 * b + k] - m1 - xh * m2);
      }
      *reinterpret_cast<floatx4*>(g_a + row * ldo + co + NPL * lane + 4 * b) = o;
    }
    return;
  }
#pragma unroll
  for (int k = 0; k < NPL; ++k) {
    const int i = NPL * lane + k;
    if (i >= n) continue;
    const float xh = (av[k] - mean) * rstd;
    g_a[row * ldo + co + i] = rstd * (gy[k] - m1 - xh * m2);
  }
}

// ------------------------------------------------------------------ RMSNormSH (lmax = 2)
__device__ __forceinline__ int deg_of(int j) { return j == 0 ? 0 : (j < 4 ? 1 : 2); }
__device__ __forceinline__ float bdw_of(int j) {
  // 1 / (2l+1) / (lmax+1), rounded from double as the reference's torch.tensor([...]) does
  const int l = deg_of(j);
  return (float)(1.0 / (2 * l + 1) / 3.0);
}

// norm.py:59-111 / mirror.py:64-75: center coefficient 0 over channels; ms = mean_c(sum_j
// bdw_j xc_j^2); inv = rsqrt(ms + eps); y = xc * (inv * aw[l(j)]); y[0] += ab (+ add0).
// One wave per node; inv[n] is kept for the backward.
__global__ __launch_bounds__(256) void k_rmsnorm_sh_fwd(const float* __restrict__ x,
                                                        const float* __restrict__ aw,
                                                        const float* __restrict__ ab,
                                                        const float* __restrict__ add0,
                                                        float* __restrict__ y,
                                                        float* __restrict__ inv_out, int64_t N,
                                                        int C, float eps) {
  const int64_t n = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
  const int lane = threadIdx.x & 63;
  if (n >= N) return;
  const float* xn = x + n * 9 * C;
  float s0 = 0.f;
  for (int c = lane; c < C; c += 64) s0 += xn[c];
  const float mu = tta_group_sum(s0, 64) / C;
  float ms = 0.f;
  for (int c = lane; c < C; c += 64) {
    float sc = 0.f;
#pragma unroll
    for (int j = 0; j < 9; ++j) {
      const float v = j == 0 ? xn[c] - mu : xn[j * C + c];
      sc += v * v * bdw_of(j);
    }
    ms += sc;
  }
  ms = tta_group_sum(ms, 64) / C;
  const float inv = 1.0f / sqrtf(ms + eps);
  if (lane == 0 && inv_out) inv_out[n] = inv;
  float* yn = y + n * 9 * C;
  for (int c = lane; c < C; c += 64) {
#pragma unroll
    for (int j = 0; j < 9; ++j) {
      const float v = j == 0 ? xn[c] - mu : xn[j * C + c];
      float o = v * (inv * aw[deg_of(j) * C + c]);
      if (j == 0) {
        o = o + ab[c];
        if (add0) o = o + add0[n * C + c];
      }
      yn[j * C + c] = o;
    }
  }
}

// Register-resident form of the RMSNormSH backward for C <= 64 NPL: each lane loads its NPL
// channels of all 9 coefficient rows of g and x (and of the 3 degree weights) once and every pass
// works from registers, so a node costs one memory round trip instead of one per pass (C3: 15 vs
// 26 us per launch).  The sums run in the same order as the loop form (channel blocks k = 0.. in
// turn, coefficients inside).  The forward keeps its loop form, which measured faster (7.2 vs
// 8.6 us): its re-reads of the row hit in cache.
template <int NPL>
__global__ __launch_bounds__(256) void k_rmsnorm_sh_bwd_r(const float* __restrict__ g,
                                                          const float* __restrict__ x,
                                                          const float* __restrict__ aw,
                                                          const float* __restrict__ inv_in,
                                                          const float* __restrict__ res,
                                                          float* __restrict__ out, int64_t N,
                                                          int C) {
  const int64_t n = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
  const int lane = threadIdx.x & 63;
  if (n >= N) return;
  const float* xn = x + n * 9 * C;
  const float* gn = g + n * 9 * C;
  float xv[9][NPL], gv[9][NPL], wv[3][NPL];
#pragma unroll
  for (int k = 0; k < NPL; ++k) {
    const int c = lane + 64 * k;
    const bool in = c < C;
#pragma unroll
    for (int j = 0; j < 9; ++j) {
      xv[j][k] = in ? xn[j * C + c] : 0.f;
      gv[j][k] = in ? gn[j * C + c] : 0.f;
    }
#pragma unroll
    for (int l = 0; l < 3; ++l) wv[l][k] = in ? aw[l * C + c] : 0.f;
  }
  const float inv = inv_in[n];
  float s0 = 0.f;
#pragma unroll
  for (int k = 0; k < NPL; ++k)
    if (lane + 64 * k < C) s0 += xv[0][k];
  const float mu = tta_group_sum(s0, 64) / C;
  float ginv = 0.f;
#pragma unroll
  for (int k = 0; k < NPL; ++k) {
    if (lane + 64 * k >= C) continue;
#pragma unroll
    for (int j = 0; j < 9; ++j) {
      const float v = j == 0 ? xv[0][k] - mu : xv[j][k];
      ginv += gv[j][k] * v * wv[deg_of(j)][k];
    }
  }
  ginv = tta_group_sum(ginv, 64);
  const float gms = ginv * (inv * inv * inv) * -0.5f;
  float s1 = 0.f;
#pragma unroll
  for (int k = 0; k < NPL; ++k) {
    if (lane + 64 * k >= C) continue;
    const float v = xv[0][k] - mu;
    s1 += gv[0][k] * (inv * wv[0][k]) + v * bdw_of(0) * gms * (2.0f / C);
  }
  const float m0 = tta_group_sum(s1, 64) / C;
  float* on = out + n * 9 * C;
#pragma unroll
  for (int k = 0; k < NPL; ++k) {
    const int c = lane + 64 * k;
    if (c >= C) continue;
#pragma unroll
    for (int j = 0; j < 9; ++j) {
      const float v = j == 0 ? xv[0][k] - mu : xv[j][k];
      float gx = gv[j][k] * (inv * wv[deg_of(j)][k]) + v * bdw_of(j) * gms * (2.0f / C);
      if (j == 0) gx -= m0;
      if (res) gx += res[n * 9 * C + j * C + c];
      on[j * C + c] = gx;
    }
  }
}

// forces.py:73-98 (VJP of RMSNormSH) + optional residual adjoint: out = g_x + res.
__global__ __launch_bounds__(256) void k_rmsnorm_sh_bwd(const float* __restrict__ g,
                                                        const float* __restrict__ x,
                                                        const float* __restrict__ aw,
                                                        const float* __restrict__ inv_in,
                                                        const float* __restrict__ res,
                                                        float* __restrict__ out, int64_t N,
                                                        int C) {
  const int64_t n = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
  const int lane = threadIdx.x & 63;
  if (n >= N) return;
  const float* xn = x + n * 9 * C;
  const float* gn = g + n * 9 * C;
  const float inv = inv_in[n];
  float s0 = 0.f;
  for (int c = lane; c < C; c += 64) s0 += xn[c];
  const float mu = tta_group_sum(s0, 64) / C;
  float ginv = 0.f;
  for (int c = lane; c < C; c += 64) {
#pragma unroll
    for (int j = 0; j < 9; ++j) {
      const float v = j == 0 ? xn[c] - mu : xn[j * C + c];
      ginv += gn[j * C + c] * v * aw[deg_of(j) * C + c];
    }
  }
  ginv = tta_group_sum(ginv, 64);
  const float gms = ginv * (inv * inv * inv) * -0.5f;
  // l0 centering backward needs mean_c of g_xc[0]
  float s1 = 0.f;
  for (int c = lane; c < C; c += 64) {
    const float v = xn[c] - mu;
    s1 += gn[c] * (inv * aw[c]) + v * bdw_of(0) * gms * (2.0f / C);
  }
  const float m0 = tta_group_sum(s1, 64) / C;
  float* on = out + n * 9 * C;
  for (int c = lane; c < C; c += 64) {
#pragma unroll
    for (int j = 0; j < 9; ++j) {
      const float v = j == 0 ? xn[c] - mu : xn[j * C + c];
      float gx = gn[j * C + c] * (inv * aw[deg_of(j) * C + c]) + v * bdw_of(j) * gms * (2.0f / C);
      if (j == 0) gx -= m0;
      if (res) gx += res[n * 9 * C + j * C + c];
      on[j * C + c] = gx;
    }
  }
}

// ------------------------------------------------------------------ elementwise / reductions
__global__ __launch_bounds__(256) void k_silu_bwd(const float* __restrict__ g,
                                                  const float* __restrict__ x,
                                                  float* __restrict__ out, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) out[i] = g[i] * tta_silu_grad(x[i]);
}

// Deterministic sum of n values with stride `stride` (single block, fixed order tree).
__global__ __launch_bounds__(1024) void k_sum(const float* __restrict__ x, int64_t n,
                                              int64_t stride, float* __restrict__ out) {
  __shared__ float part[16];
  float s = 0.f;
  for (int64_t i = threadIdx.x; i < n; i += 1024) s += x[i * stride];
  s = tta_group_sum(s, 64);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = s;
  __syncthreads();
  if (threadIdx.x < 64) {
    float v = threadIdx.x < 16 ? part[threadIdx.x] : 0.f;
    v = tta_group_sum(v, 64);
    if (threadIdx.x == 0) out[0] = v;
  }
}

// Per-segment sums of x over the contiguous ranges [ptr[k], ptr[k+1]), one block per segment,
// each with exactly k_sum's order (so a system's sum inside a batch equals its sum alone).
__global__ __launch_bounds__(1024) void k_segment_sum(const float* __restrict__ x,
                                                      const int* __restrict__ ptr,
                                                      float* __restrict__ out) {
  __shared__ float part[16];
  const int k = blockIdx.x;
  const float* xs = x + ptr[k];
  const int64_t n = ptr[k + 1] - ptr[k];
  float s = 0.f;
  for (int64_t i = threadIdx.x; i < n; i += 1024) s += xs[i];
  s = tta_group_sum(s, 64);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = s;
  __syncthreads();
  if (threadIdx.x < 64) {
    float v = threadIdx.x < 16 ? part[threadIdx.x] : 0.f;
    v = tta_group_sum(v, 64);
    if (threadIdx.x == 0) out[k] = v;
  }
}

// out[r, c] = value for all c in [0, n): used to seed the energy adjoint with ones.
__global__ __launch_bounds__(256) void k_fill(float* __restrict__ out, int64_t n, float value) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) out[i] = value;
}

}  // namespace

extern "C" int tta_gate_fwd(const float* x, const float* gating, float* y, int64_t R, int64_t H,
                            int64_t L, int64_t ldx, int64_t ldg, const int* idx8,
                            hipStream_t stream) {
  TTA_CHECK_ARG(R >= 0 && H > 0 && L >= 1 && L <= 8, "tta_gate_fwd: bad sizes");
  TTA_CHECK_ARG(ldx >= 9 * H && ldg >= L * H, "tta_gate_fwd: row stride too small");
  TTA_CHECK_ARG(idx8, "tta_gate_fwd: null index table");
  GateIdx gi;
  for (int i = 0; i < 8; ++i) {
    TTA_CHECK_ARG(idx8[i] >= 0 && idx8[i] < L, "tta_gate_fwd: gate index out of range");
    gi.v[i] = idx8[i];
  }
  if (R == 0) return tta::kOk;
  TTA_CHECK_ARG(x && gating && y, "tta_gate_fwd: null pointer");
  hipLaunchKernelGGL(k_gate_fwd, dim3(tta_blocks(R * H, 256)), dim3(256), 0, stream, x, gating, y,
                     R, (int)H, (int)L, ldx, ldg, gi);
  TTA_CHECK_LAUNCH("tta_gate_fwd");
  return tta::kOk;
}

extern "C" int tta_gate_bwd(const float* g_y, const float* x, const float* gating, float* g_x,
                            float* g_gating, int64_t R, int64_t H, int64_t L, int64_t ldx,
                            int64_t ldg, const int* idx8, hipStream_t stream) {
  TTA_CHECK_ARG(R >= 0 && H > 0 && L >= 1 && L <= 8, "tta_gate_bwd: bad sizes");
  TTA_CHECK_ARG(ldx >= 9 * H && ldg >= L * H, "tta_gate_bwd: row stride too small");
  TTA_CHECK_ARG(idx8, "tta_gate_bwd: null index table");
  GateIdx gi;
  for (int i = 0; i < 8; ++i) {
    TTA_CHECK_ARG(idx8[i] >= 0 && idx8[i] < L, "tta_gate_bwd: gate index out of range");
    gi.v[i] = idx8[i];
  }
  if (R == 0) return tta::kOk;
  TTA_CHECK_ARG(g_y && x && gating && g_x && g_gating, "tta_gate_bwd: null pointer");
  hipLaunchKernelGGL(k_gate_bwd, dim3(tta_blocks(R * H, 256)), dim3(256), 0, stream, g_y, x,
                     gating, g_x, g_gating, R, (int)H, (int)L, ldx, ldg, gi);
  TTA_CHECK_LAUNCH("tta_gate_bwd");
  return tta::kOk;
}

extern "C" int tta_gate_gating_bwd(const float* g_x, const float* y, const float* sig,
                                   float* g_gating, int64_t R, int64_t H, int64_t L,
                                   int64_t ldgx, int64_t ldg, int64_t ldgg, const int* idx8,
                                   hipStream_t stream) {
  TTA_CHECK_ARG(R >= 0 && H > 0 && L >= 1 && L <= 8, "tta_gate_gating_bwd: bad sizes");
  TTA_CHECK_ARG(ldgx >= 9 * H && ldg >= L * H && ldgg >= L * H,
                "tta_gate_gating_bwd: row stride too small");
  TTA_CHECK_ARG(idx8, "tta_gate_gating_bwd: null index table");
  GateIdx gi;
  for (int i = 0; i < 8; ++i) {
    TTA_CHECK_ARG(idx8[i] >= 0 && idx8[i] < L, "tta_gate_gating_bwd: gate index out of range");
    gi.v[i] = idx8[i];
  }
  if (R == 0) return tta::kOk;
  TTA_CHECK_ARG(g_x && y && sig && g_gating, "tta_gate_gating_bwd: null pointer");
  hipLaunchKernelGGL(k_gate_gating_bwd, dim3(tta_blocks(R * H, 256)), dim3(256), 0, stream, g_x,
                     y, sig, g_gating, R, (int)H, (int)L, ldgx, ldg, ldgg, gi);
  TTA_CHECK_LAUNCH("tta_gate_gating_bwd");
  return tta::kOk;
}

// a null pointer counts as aligned (an operand the call does not use)
static bool al16(const void* q) { return ((uintptr_t)q & 15) == 0; }

extern "C" int tta_ln_silu_fwd(const float* a, const float* gamma, const float* beta, float* nrm,
                               float* s, int64_t R, int64_t n, int64_t groups, int64_t lda,
                               int64_t lds, float eps, hipStream_t stream) {
  TTA_CHECK_ARG(R >= 0 && n > 0 && n <= 512 && groups >= 1 && groups <= 64 &&
                    lda >= groups * n && lds >= groups * n && R * groups < ((int64_t)1 << 40),
                "tta_ln_silu_fwd: bad sizes (row width 1..512, 1..64 groups)");
  if (R == 0) return tta::kOk;
  TTA_CHECK_ARG(a && gamma && beta && s, "tta_ln_silu_fwd: null pointer");
  const int64_t RV = R * groups;
  // float4 rows (four contiguous columns per lane) when a row group is exactly four per lane and
  // every row starts 16-byte aligned
  const bool vec = (n == 128 || n == 256) && lda % 4 == 0 && lds % 4 == 0 && al16(a) &&
                   al16(gamma) && al16(beta) && al16(nrm) && al16(s);
#define TTA_LN_FWD(G, NPL, VEC)                                                             \
  hipLaunchKernelGGL((k_ln_silu_fwd<G, NPL, VEC>), dim3(tta_blocks(RV * G, 256)), dim3(256),  \
                     0, stream, a, gamma, beta, nrm, s, R, (int)n, (int)groups, lda, lds, eps)
  if (n <= 32)
    TTA_LN_FWD(32, 1, false);
  else if (n <= 64)
    TTA_LN_FWD(32, 2, false);
  else if (n <= 128 && vec)
    TTA_LN_FWD(16, 8, true);
  else if (n <= 128)
    TTA_LN_FWD(16, 8, false);
  else if (n <= 256 && vec)
    TTA_LN_FWD(64, 4, true);
  else if (n <= 256)
    TTA_LN_FWD(64, 4, false);
  else
    TTA_LN_FWD(64, 8, false);
#undef TTA_LN_FWD
  TTA_CHECK_LAUNCH("tta_ln_silu_fwd");
  return tta::kOk;
}

extern "C" int tta_ln_silu_bwd(const float* g, const float* a, const float* nrm,
                               const float* gamma, const float* beta, float* g_a, int64_t R,
                               int64_t n, int64_t groups, int64_t ldg, int64_t lda, int64_t ldo,
                               float eps, hipStream_t stream) {
  TTA_CHECK_ARG(R >= 0 && n > 0 && n <= 512 && groups >= 1 && groups <= 64 &&
                    ldg >= groups * n && lda >= groups * n && ldo >= groups * n &&
                    R * groups < ((int64_t)1 << 40),
                "tta_ln_silu_bwd: bad sizes (row width 1..512, 1..64 groups)");
  if (R == 0) return tta::kOk;
  TTA_CHECK_ARG(g && a && gamma && g_a && (nrm || beta),
                "tta_ln_silu_bwd: null pointer (nrm, or beta to recompute it, is required)");
  const int64_t RV = R * groups;
  const bool vec = (n == 128 || n == 256) && ldg % 4 == 0 && lda % 4 == 0 && ldo % 4 == 0 &&
                   al16(g) && al16(a) && al16(nrm) && al16(gamma) && al16(beta) && al16(g_a);
#define TTA_LN_BWD(G, NPL, VEC)                                                             \
  do {                                                                                      \
    if (nrm)                                                                                \
      hipLaunchKernelGGL((k_ln_silu_bwd<G, NPL, false, VEC>), dim3(tta_blocks(RV * G, 256)), \
                         dim3(256), 0, stream, g, a, nrm, gamma, beta, g_a, R, (int)n,      \
                         (int)groups, ldg, lda, ldo, eps);                                  \
    else                                                                                    \
      hipLaunchKernelGGL((k_ln_silu_bwd<G, NPL, true, VEC>), dim3(tta_blocks(RV * G, 256)), \
                         dim3(256), 0, stream, g, a, nrm, gamma, beta, g_a, R, (int)n,      \
                         (int)groups, ldg, lda, ldo, eps);                                  \
  } while (0)
  if (n <= 32)
    TTA_LN_BWD(32, 1, false);
  else if (n <= 64)
    TTA_LN_BWD(32, 2, false);
  else if (n <= 128 && vec)
    TTA_LN_BWD(16, 8, true);
  else if (n <= 128)
    TTA_LN_BWD(16, 8, false);
  else if (n <= 256 && vec)
    TTA_LN_BWD(64, 4, true);
  else if (n <= 256)
    TTA_LN_BWD(64, 4, false);
  else
    TTA_LN_BWD(64, 8, false);
#undef TTA_LN_BWD
  TTA_CHECK_LAUNCH("tta_ln_silu_bwd");
  return tta::kOk;
}

extern "C" int tta_rmsnorm_sh_fwd(const float* x, const float* aw, const float* ab,
                                  const float* add0, float* y, float* inv, int64_t N, int64_t C,
                                  float eps, hipStream_t stream) {
  TTA_CHECK_ARG(N >= 0 && C > 0, "tta_rmsnorm_sh_fwd: bad sizes");
  if (N == 0) return tta::kOk;
  TTA_CHECK_ARG(x && aw && ab && y, "tta_rmsnorm_sh_fwd: null pointer");
  hipLaunchKernelGGL(k_rmsnorm_sh_fwd, dim3(tta_blocks(N * 64, 256)), dim3(256), 0, stream, x, aw,
                     ab, add0, y, inv, N, (int)C, eps);
  TTA_CHECK_LAUNCH("tta_rmsnorm_sh_fwd");
  return tta::kOk;
}

extern "C" int tta_rmsnorm_sh_bwd(const float* g, const float* x, const float* aw,
                                  const float* inv, const float* res, float* out, int64_t N,
                                  int64_t C, hipStream_t stream) {
  TTA_CHECK_ARG(N >= 0 && C > 0, "tta_rmsnorm_sh_bwd: bad sizes");
  if (N == 0) return tta::kOk;
  TTA_CHECK_ARG(g && x && aw && inv && out, "tta_rmsnorm_sh_bwd: null pointer");
  const dim3 grid(tta_blocks(N * 64, 256));
  if (C <= 64)
    hipLaunchKernelGGL(k_rmsnorm_sh_bwd_r<1>, grid, dim3(256), 0, stream, g, x, aw, inv, res, out,
                       N, (int)C);
  else if (C <= 128)
    hipLaunchKernelGGL(k_rmsnorm_sh_bwd_r<2>, grid, dim3(256), 0, stream, g, x, aw, inv, res, out,
                       N, (int)C);
  else if (C <= 256)
    hipLaunchKernelGGL(k_rmsnorm_sh_bwd_r<4>, grid, dim3(256), 0, stream, g, x, aw, inv, res, out,
                       N, (int)C);
  else
    hipLaunchKernelGGL(k_rmsnorm_sh_bwd, grid, dim3(256), 0, stream, g, x, aw, inv, res, out, N,
                       (int)C);
  TTA_CHECK_LAUNCH("tta_rmsnorm_sh_bwd");
  return tta::kOk;
}

extern "C" int tta_silu_bwd(const float* g, const float* x, float* out, int64_t n,
                            hipStream_t stream) {
  TTA_CHECK_ARG(n >= 0, "tta_silu_bwd: bad size");
  if (n == 0) return tta::kOk;
  TTA_CHECK_ARG(g && x && out, "tta_silu_bwd: null pointer");
  hipLaunchKernelGGL(k_silu_bwd, dim3(tta_blocks(n, 256)), dim3(256), 0, stream, g, x, out, n);
  TTA_CHECK_LAUNCH("tta_silu_bwd");
  return tta::kOk;
}

extern "C" int tta_sum(const float* x, int64_t n, int64_t stride, float* out,
                       hipStream_t stream) {
  TTA_CHECK_ARG(n >= 0 && stride >= 1, "tta_sum: bad size");
  TTA_CHECK_ARG(out && (x || n == 0), "tta_sum: null pointer");
  hipLaunchKernelGGL(k_sum, dim3(1), dim3(1024), 0, stream, x, n, stride, out);
  TTA_CHECK_LAUNCH("tta_sum");
  return tta::kOk;
}

extern "C" int tta_segment_sum(const float* x, const int* ptr, int64_t K, float* out,
                               hipStream_t stream) {
  TTA_CHECK_ARG(K >= 0 && K <= 0x7fffffff, "tta_segment_sum: bad segment count");
  if (K == 0) return tta::kOk;
  TTA_CHECK_ARG(x && ptr && out, "tta_segment_sum: null pointer");
  hipLaunchKernelGGL(k_segment_sum, dim3((unsigned)K), dim3(1024), 0, stream, x, ptr, out);
  TTA_CHECK_LAUNCH("tta_segment_sum");
  return tta::kOk;
}

extern "C" int tta_fill(float* out, int64_t n, float value, hipStream_t stream) {
  TTA_CHECK_ARG(n >= 0, "tta_fill: bad size");
  if (n == 0) return tta::kOk;
  TTA_CHECK_ARG(out, "tta_fill: null pointer");
  hipLaunchKernelGGL(k_fill, dim3(tta_blocks(n, 256)), dim3(256), 0, stream, out, n, value);
  TTA_CHECK_LAUNCH("tta_fill");
  return tta::kOk;
}
