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

// The z-rotation block of degree L (size n = 2L+1, geometry.py:124-136) is sparse: row i holds
// cos(f t) at column i and sin(f t) at column n-1-i, f = L - i, and the centre row is exactly 1
// (cos 0 + sin 0).  Its entries are the cosines and sines of t and 2t only, so one ZTrig per
// angle serves both degrees, and products with a Z block touch two terms per entry instead of n.
struct ZTrig {
  float c[3], s[3];  // cos(k t), sin(k t), k = 0, 1, 2
};

TTA_HD ZTrig ztrig(float t) {
  ZTrig z;
  z.c[0] = 1.f;
  z.s[0] = 0.f;
  z.c[1] = cosf(t);
  z.s[1] = sinf(t);
  z.c[2] = cosf(2.f * t);
  z.s[2] = sinf(2.f * t);
  return z;
}

TTA_HD float zcos(const ZTrig& z, int f) { return z.c[f < 0 ? -f : f]; }
TTA_HD float zsin(const ZTrig& z, int f) { return f < 0 ? -z.s[-f] : z.s[f]; }

// out = Z M (n x n, row-major); the two terms of each entry are added in column order of Z.
template <int L>
TTA_HD void zleft(const ZTrig& z, const float* M, float* out) {
  constexpr int n = 2 * L + 1;
#pragma unroll
  for (int i = 0; i < n; ++i) {
    const int f = L - i, i2 = n - 1 - i;
#pragma unroll
    for (int j = 0; j < n; ++j) {
      if (f == 0) {
        out[i * n + j] = M[i * n + j];
      } else {
        const float d = zcos(z, f) * M[i * n + j], a = zsin(z, f) * M[i2 * n + j];
        out[i * n + j] = i < i2 ? d + a : a + d;
      }
    }
  }
}

// out = M Z; column j of Z holds cos(f_j t) at row j and sin(-f_j t) at row n-1-j.
template <int L>
TTA_HD void zright(const ZTrig& z, const float* M, float* out) {
  constexpr int n = 2 * L + 1;
#pragma unroll
  for (int j = 0; j < n; ++j) {
    const int f = L - j, j2 = n - 1 - j;
#pragma unroll
    for (int i = 0; i < n; ++i) {
      if (f == 0) {
        out[i * n + j] = M[i * n + j];
      } else {
        const float d = M[i * n + j] * zcos(z, f), a = M[i * n + j2] * zsin(z, -f);
        out[i * n + j] = j < j2 ? d + a : a + d;
      }
    }
  }
}

template <int n>
TTA_HD void matmul(const float* A, const float* B, float* C) {
#pragma unroll
  for (int i = 0; i < n; ++i)
#pragma unroll
    for (int j = 0; j < n; ++j) {
      float s = 0.f;
#pragma unroll
      for (int k = 0; k < n; ++k) s += A[i * n + k] * B[k * n + j];
      C[i * n + j] = s;
    }
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

// D = ((((Za J) Zb) J) Zc), the torch evaluation order of geometry.py:142, with the Z products
// taken sparse (the dense products add exact zeros).
template <int L>
TTA_HD void wigner_block(const float* J, const ZTrig& za, const ZTrig& zb, const ZTrig& zc,
                         float* D) {
  constexpr int n = 2 * L + 1;
  float T1[n * n], T2[n * n];
  zleft<L>(za, J, T1);
  zright<L>(zb, T1, T2);
  matmul<n>(T2, J, T1);
  zright<L>(zc, T1, D);
}

// Packed Wigner coefficients [35] of one edge.  jd = [Jd_0 (1) | Jd_1 (9) | Jd_2 (25)].
TTA_HD void wigner_coef(const float ev[3], float gamma, const float* jd, float* coef) {
  const Frame f = frame_of(ev, gamma);
  const ZTrig za = ztrig(f.alpha_u), zb = ztrig(f.beta_u), zc = ztrig(f.gamma_u);
  // l = 0: D = Za J Zb J Zc with 1x1 blocks; every Z_0 is exactly 1.
  coef[0] = ((jd[0] * 1.f) * 1.f * jd[0]) * 1.f;
  {
    float D[9];
    wigner_block<1>(jd + 1, za, zb, zc, D);
    for (int r = 0; r < 3; ++r)
      for (int q = 0; q < 3; ++q) coef[row_koff_l1(r) + q] = D[r * 3 + q];
  }
  {
    float D[25];
    wigner_block<2>(jd + 10, za, zb, zc, D);
    for (int r = 0; r < 5; ++r)
      for (int q = 0; q < 5; ++q) coef[row_koff_l2(r) + q] = D[r * 5 + q];
  }
}

// sum_ij G_ij d D_ij / d(beta_u) and d D_ij / d(gamma_u) for one degree block, D = A Zb J Zc with
// A = Za J.  By the cyclic trace,
//   gb = sum_kl dZb_kl (A^T G B^T)_kl,  B = J Zc,
//   gc = sum_kl dZc_kl (R^T G)_kl,      R = A Zb J,
// and dZ (d/dt of Z) is nonzero only at (k, k) = -f sin(f t) and (k, n-1-k) = f cos(f t), so
// only those 2(n-1) entries of the two n x n products are formed.
template <int L>
TTA_HD void block_angle_grads(const float* J, const ZTrig& za, const ZTrig& zb, const ZTrig& zc,
                              const float* G, float& gb, float& gc) {
  constexpr int n = 2 * L + 1;
  float A[n * n], T[n * n], R[n * n];
  zleft<L>(za, J, A);
  zright<L>(zb, A, T);
  matmul<n>(T, J, R);
#pragma unroll
  for (int k = 0; k < n; ++k) {
    const int f = L - k, k2 = n - 1 - k;
    if (f == 0) continue;
    float dd = 0.f, da = 0.f;  // (R^T G)_{k,k}, (R^T G)_{k,k2}
#pragma unroll
    for (int i = 0; i < n; ++i) {
      dd += R[i * n + k] * G[i * n + k];
      da += R[i * n + k] * G[i * n + k2];
    }
    gc += (-(float)f * zsin(zc, f)) * dd + ((float)f * zcos(zc, f)) * da;
  }
  zright<L>(zc, J, T);  // B = J Zc
  // P = G B^T, reusing R
#pragma unroll
  for (int i = 0; i < n; ++i)
#pragma unroll
    for (int l = 0; l < n; ++l) {
      float s = 0.f;
#pragma unroll
      for (int j = 0; j < n; ++j) s += G[i * n + j] * T[l * n + j];
      R[i * n + l] = s;
    }
#pragma unroll
  for (int k = 0; k < n; ++k) {
    const int f = L - k, k2 = n - 1 - k;
    if (f == 0) continue;
    float dd = 0.f, da = 0.f;  // (A^T P)_{k,k}, (A^T P)_{k,k2}
#pragma unroll
    for (int i = 0; i < n; ++i) {
      dd += A[i * n + k] * R[i * n + k];
      da += A[i * n + k] * R[i * n + k2];
    }
    gb += (-(float)f * zsin(zb, f)) * dd + ((float)f * zcos(zb, f)) * da;
  }
}

// VJP of wigner_coef: given g_coef[35] returns g_ev[3] (adds into g_ev).
TTA_HD void wigner_vjp(const float ev[3], float gamma, const float* jd, const float* gcoef,
                       float g_ev[3]) {
  const Frame f = frame_of(ev, gamma);
  const ZTrig za = ztrig(f.alpha_u), zb = ztrig(f.beta_u), zc = ztrig(f.gamma_u);
  float gb = 0.f, gc = 0.f;
  {
    float G[9];
    for (int r = 0; r < 3; ++r)
      for (int q = 0; q < 3; ++q) G[r * 3 + q] = gcoef[row_koff_l1(r) + q];
    block_angle_grads<1>(jd + 1, za, zb, zc, G, gb, gc);
  }
  {
    float G[25];
    for (int r = 0; r < 5; ++r)
      for (int q = 0; q < 5; ++q) G[r * 5 + q] = gcoef[row_koff_l2(r) + q];
    block_angle_grads<2>(jd + 10, za, zb, zc, G, gb, gc);
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
