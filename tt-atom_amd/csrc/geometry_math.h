// Per-edge geometry math of the eSCN-MD path, shared by the gfx950 kernels and a host build used
// by the CPU tests: the Wigner-D rotation into the edge frame (lmax = 2, gamma gauge) in the
// packed 35-coefficient layout, and its closed-form vector-Jacobian product back to the edge
// vector, reproducing the reference's regularised acos / atan2 gradients.
//
// Reference: tt_atom/geometry.py:87-155 (Euler angles, z-rotations, D = Z(a) J Z(b) J Z(c)),
// geometry.py:209-224 (the to_m row permutation [0,2,6,3,7,1,5,8,4]), rotation.py:196-208 (pack
// order).
#pragma once

#include <math.h>

#if defined(__HIPCC__)
#define TTA_HD __host__ __device__ __forceinline__
#else
#define TTA_HD inline
#endif

namespace tta_geo {

constexpr float kEps = 1e-7f;          // geometry.py:20
constexpr float kNormEps = 1e-12f;     // F.normalize default eps

// Packed-coefficient offset of the m-primed Wigner row stored at each local row of the l = 1
// and l = 2 blocks (natural rows 1..3 and 4..8).  Natural row perm[m] holds m-primed row m.
TTA_HD int row_koff_l1(int r) { return r == 0 ? 17 : (r == 1 ? 1 : 9); }
TTA_HD int row_koff_l2(int r) {
  return r == 0 ? 30 : (r == 1 ? 20 : (r == 2 ? 4 : (r == 3 ? 12 : 25)));
}

// Dense z-rotation block of degree l (size n = 2l+1): Z[i][i] = cos(f_i t), Z[i][n-1-i] =
// sin(f_i t), f_i = l - i (geometry.py:124-136; the centre is cos(0) + sin(0) = 1).
template <int L>
TTA_HD void zrot(float t, float* Z) {
  constexpr int n = 2 * L + 1;
  for (int i = 0; i < n * n; ++i) Z[i] = 0.f;
  for (int i = 0; i < n; ++i) {
    const float fa = (float)(L - i) * t;
    Z[i * n + i] += cosf(fa);
    Z[i * n + (n - 1 - i)] += sinf(fa);
  }
}

// d Z / d t
template <int L>
TTA_HD void zrot_d(float t, float* Z) {
  constexpr int n = 2 * L + 1;
  for (int i = 0; i < n * n; ++i) Z[i] = 0.f;
  for (int i = 0; i < n; ++i) {
    const float f = (float)(L - i);
    const float fa = f * t;
    Z[i * n + i] += -f * sinf(fa);
    Z[i * n + (n - 1 - i)] += f * cosf(fa);
  }
}

template <int n>
TTA_HD void matmul(const float* A, const float* B, float* C) {
  for (int i = 0; i < n; ++i)
    for (int j = 0; j < n; ++j) {
      float s = 0.f;
      for (int k = 0; k < n; ++k) s += A[i * n + k] * B[k * n + j];
      C[i * n + j] = s;
    }
}

// D = ((((Za J) Zb) J) Zc), the torch evaluation order of geometry.py:142.
template <int L>
TTA_HD void wigner_block(const float* J, const float* Za, const float* Zb, const float* Zc,
                         float* D) {
  constexpr int n = 2 * L + 1;
  float T1[n * n], T2[n * n];
  matmul<n>(Za, J, T1);
  matmul<n>(T1, Zb, T2);
  matmul<n>(T2, J, T1);
  matmul<n>(T1, Zc, D);
}

struct Frame {
  float n;          // |ev|
  float u[3];       // clamp(normalize(ev), -1, 1)
  float uraw[3];    // normalize(ev) before the clamp
  float alpha_u, beta_u, gamma_u;  // angles fed to D (geometry.py:112-118: -gamma, -beta, -alpha)
};

TTA_HD Frame frame_of(const float ev[3], float gamma) {
  Frame f;
  f.n = sqrtf(ev[0] * ev[0] + ev[1] * ev[1] + ev[2] * ev[2]);
  const float nc = f.n > kNormEps ? f.n : kNormEps;
  for (int k = 0; k < 3; ++k) {
    f.uraw[k] = ev[k] / nc;
    f.u[k] = fminf(fmaxf(f.uraw[k], -1.f), 1.f);
  }
  const float beta = acosf(f.u[1]);
  const float alpha = atan2f(f.u[0], f.u[2]);
  f.alpha_u = -gamma;
  f.beta_u = -beta;
  f.gamma_u = -alpha;
  return f;
}

// Packed Wigner coefficients [35] of one edge.  jd = [Jd_0 (1) | Jd_1 (9) | Jd_2 (25)].
TTA_HD void wigner_coef(const float ev[3], float gamma, const float* jd, float* coef) {
  const Frame f = frame_of(ev, gamma);
  // l = 0: D = Za J Zb J Zc with 1x1 blocks; every Z_0 is exactly 1.
  coef[0] = ((jd[0] * 1.f) * 1.f * jd[0]) * 1.f;
  {
    float Za[9], Zb[9], Zc[9], D[9];
    zrot<1>(f.alpha_u, Za);
    zrot<1>(f.beta_u, Zb);
    zrot<1>(f.gamma_u, Zc);
    wigner_block<1>(jd + 1, Za, Zb, Zc, D);
    for (int r = 0; r < 3; ++r)
      for (int q = 0; q < 3; ++q) coef[row_koff_l1(r) + q] = D[r * 3 + q];
  }
  {
    float Za[25], Zb[25], Zc[25], D[25];
    zrot<2>(f.alpha_u, Za);
    zrot<2>(f.beta_u, Zb);
    zrot<2>(f.gamma_u, Zc);
    wigner_block<2>(jd + 10, Za, Zb, Zc, D);
    for (int r = 0; r < 5; ++r)
      for (int q = 0; q < 5; ++q) coef[row_koff_l2(r) + q] = D[r * 5 + q];
  }
}

// sum_ij G_ij d D_ij / d(beta_u), d(gamma_u) for one degree block.
template <int L>
TTA_HD void block_angle_grads(const float* J, const Frame& f, const float* G, float& gb,
                              float& gc) {
  constexpr int n = 2 * L + 1;
  float Za[n * n], Zb[n * n], Zc[n * n], dZ[n * n], D[n * n];
  zrot<L>(f.alpha_u, Za);
  zrot<L>(f.beta_u, Zb);
  zrot<L>(f.gamma_u, Zc);
  zrot_d<L>(f.beta_u, dZ);
  wigner_block<L>(J, Za, dZ, Zc, D);
  for (int i = 0; i < n * n; ++i) gb += G[i] * D[i];
  zrot_d<L>(f.gamma_u, dZ);
  wigner_block<L>(J, Za, Zb, dZ, D);
  for (int i = 0; i < n * n; ++i) gc += G[i] * D[i];
}

// VJP of wigner_coef: given g_coef[35] returns g_ev[3] (adds into g_ev).
TTA_HD void wigner_vjp(const float ev[3], float gamma, const float* jd, const float* gcoef,
                       float g_ev[3]) {
  const Frame f = frame_of(ev, gamma);
  float gb = 0.f, gc = 0.f;
  {
    float G[9];
    for (int r = 0; r < 3; ++r)
      for (int q = 0; q < 3; ++q) G[r * 3 + q] = gcoef[row_koff_l1(r) + q];
    block_angle_grads<1>(jd + 1, f, G, gb, gc);
  }
  {
    float G[25];
    for (int r = 0; r < 5; ++r)
      for (int q = 0; q < 5; ++q) G[r * 5 + q] = gcoef[row_koff_l2(r) + q];
    block_angle_grads<2>(jd + 10, f, G, gb, gc);
  }
  // beta_u = -beta, gamma_u = -alpha
  const float g_beta = -gb;
  const float g_alpha = -gc;
  // SafeAcos (geometry.py:87-96): d beta / d y = -1 / clamp(sqrt(1 - yc^2), EPS)
  const float yc = fminf(fmaxf(f.u[1], -1.f + kEps), 1.f - kEps);
  float sq = sqrtf(1.f - yc * yc);
  sq = sq > kEps ? sq : kEps;
  float gu[3];
  gu[1] = -g_beta / sq;
  // SafeAtan2(y = u_x, x = u_z) (geometry.py:99-109): denom = clamp(u_z^2 + u_x^2, EPS)
  float den = f.u[2] * f.u[2] + f.u[0] * f.u[0];
  den = den > kEps ? den : kEps;
  gu[0] = g_alpha * f.u[2] / den;
  gu[2] = -g_alpha * f.u[0] / den;
  // clamp(-1, 1) passes the gradient where -1 <= u <= 1
  for (int k = 0; k < 3; ++k)
    if (!(f.uraw[k] >= -1.f && f.uraw[k] <= 1.f)) gu[k] = 0.f;
  // u = ev / max(|ev|, eps)
  const float nc = f.n > kNormEps ? f.n : kNormEps;
  float dot = 0.f;
  for (int k = 0; k < 3; ++k) dot += gu[k] * ev[k];
  for (int k = 0; k < 3; ++k) {
    float g = gu[k] / nc;
    if (f.n > kNormEps && f.n > 0.f) g -= dot / (nc * nc) * (ev[k] / f.n);
    g_ev[k] += g;
  }
}

// Radial terms of one edge: gaussian basis exp(coeff (d - off_k)^2) and the polynomial envelope
// (p = 5) of geometry.py:243-251.
TTA_HD float envelope(float d, float cutoff) {
  const float ds = d / cutoff;
  if (!(ds < 1.f)) return 0.f;
  const float a = -21.f, b = 35.f, c = -15.f;  // -(p+1)(p+2)/2, p(p+2), -p(p+1)/2 at p = 5
  const float ds2 = ds * ds;
  const float ds5 = ds2 * ds2 * ds;
  return 1.f + ds5 * (a + ds * (b + c * ds));
}

TTA_HD float envelope_grad(float d, float cutoff) {
  const float ds = d / cutoff;
  if (!(ds < 1.f)) return 0.f;
  const float a = -21.f, b = 35.f, c = -15.f;
  const float ds2 = ds * ds;
  const float ds4 = ds2 * ds2;
  const float ds5 = ds4 * ds;
  return (5.f * ds4 * (a + ds * (b + c * ds)) + ds5 * (b + 2.f * c * ds)) / cutoff;
}

}  // namespace tta_geo
