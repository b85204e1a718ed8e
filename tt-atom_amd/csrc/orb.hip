// Orb-v3 edge-MLP + scatter path on gfx950: the fixed edge descriptor (Bessel x real spherical
// harmonics x polynomial cutoff) and its closed-form force VJP, the fused RMSNorm + residual +
// attention-gate row kernel, the sender/receiver segment sums that build the node-MLP input,
// the per-edge backward that joins the scatter adjoint, the attention adjoint and the RMSNorm
// adjoint, and the node-level segment sums of the first edge-MLP layer's adjoint.
//
// Edge order is sender-sorted (stable), so sender segments are contiguous ranges
// [send_ptr[n], send_ptr[n+1]); receiver segments go through recv_perm.  Every reduction runs in
// a fixed order (no atomics), so the results are bitwise reproducible.
#include "common.h"

namespace {

typedef float floatx4 __attribute__((ext_vector_type(4)));

// ------------------------------------------------------------------------------ geometry
// Real spherical harmonics l = 0..3 of a unit vector with each l block scaled by sqrt(2l+1)
// (orb_geometry.py:37-62: e3nn component order).
__device__ __forceinline__ void sph_l3(float x, float y, float z, float* Y) {
  const float s3 = 1.7320508075688772f, s5 = 2.2360679774997896f, s7 = 2.6457513110645906f;
  const float k56 = 0.9128709291752769f;  // sqrt(5/6)
  const float k38 = 0.6123724356957945f;  // sqrt(3/8)
  const float xx = x * x, yy = y * y, zz = z * z, p = xx + zz;
  const float c20 = s3 * x * z, c24 = 0.5f * s3 * (zz - xx);
  Y[0] = 1.f;
  Y[1] = s3 * x;
  Y[2] = s3 * y;
  Y[3] = s3 * z;
  Y[4] = s5 * c20;
  Y[5] = s5 * (s3 * x * y);
  Y[6] = s5 * (yy - 0.5f * p);
  Y[7] = s5 * (s3 * y * z);
  Y[8] = s5 * c24;
  Y[9] = s7 * (k56 * (c20 * z + c24 * x));
  Y[10] = s7 * (s5 * c20 * y);
  Y[11] = s7 * (k38 * (4.f * yy - p) * x);
  Y[12] = s7 * (0.5f * y * (2.f * yy - 3.f * p));
  Y[13] = s7 * (k38 * (4.f * yy - p) * z);
  Y[14] = s7 * (s5 * c24 * y);
  Y[15] = s7 * (k56 * (c24 * z - c20 * x));
}

// d/du of sum_m gY[m] Y_m(u), treating (x, y, z) as independent (the unit-sphere projection is
// applied by the caller).  Derivatives of the unscaled harmonics:
//   l=2: sqrt3 xz, sqrt3 xy, y^2 - (x^2+z^2)/2, sqrt3 yz, sqrt3/2 (z^2 - x^2)
//   l=3: sqrt(5/2)(3/2 x z^2 - x^3/2), sqrt15 xyz, sqrt(3/8)(4y^2 - x^2 - z^2)x,
//        y^3 - 3/2 y (x^2+z^2), sqrt(3/8)(4y^2 - x^2 - z^2)z, sqrt15/2 (z^2 - x^2)y,
//        sqrt(5/2)(z^3/2 - 3/2 x^2 z)
__device__ __forceinline__ void sph_l3_vjp(float x, float y, float z, const float* gY, float& gx,
                                           float& gy, float& gz) {
  const float s3 = 1.7320508075688772f, s5 = 2.2360679774997896f, s7 = 2.6457513110645906f;
  const float s15 = 3.872983346207417f, k52 = 1.5811388300841898f, k38 = 0.6123724356957945f;
  float q[16];
  q[1] = gY[1] * s3;
  q[2] = gY[2] * s3;
  q[3] = gY[3] * s3;
#pragma unroll
  for (int m = 4; m < 9; ++m) q[m] = gY[m] * s5;
#pragma unroll
  for (int m = 9; m < 16; ++m) q[m] = gY[m] * s7;
  const float xx = x * x, yy = y * y, zz = z * z;
  gx = q[1] + s3 * (q[4] * z + q[5] * y) - q[6] * x - s3 * q[8] * x;
  gy = q[2] + s3 * q[5] * x + 2.f * q[6] * y + s3 * q[7] * z;
  gz = q[3] + s3 * q[4] * x - q[6] * z + s3 * q[7] * y + s3 * q[8] * z;
  gx += q[9] * (1.5f * k52) * (zz - xx) + q[10] * s15 * y * z +
        q[11] * k38 * (4.f * yy - 3.f * xx - zz) - q[12] * 3.f * x * y -
        q[13] * k38 * 2.f * x * z - q[14] * s15 * x * y - q[15] * (3.f * k52) * x * z;
  gy += q[10] * s15 * x * z + q[11] * k38 * 8.f * x * y + q[12] * (3.f * yy - 1.5f * (xx + zz)) +
        q[13] * k38 * 8.f * y * z + q[14] * (0.5f * s15) * (zz - xx);
  gz += q[9] * (3.f * k52) * x * z + q[10] * s15 * x * y - q[11] * k38 * 2.f * x * z -
        q[12] * 3.f * y * z + q[13] * k38 * (4.f * yy - xx - 3.f * zz) + q[14] * s15 * y * z +
        q[15] * (1.5f * k52) * (zz - xx);
}

// Polynomial cutoff p = 4 (orb_model.py:69-82): 1 - 15 q^4 + 24 q^5 - 10 q^6 for r < r_max,
// evaluated in the factored form (1 - q)^3 (1 + 3q + 6q^2 + 10q^3), which has no cancellation as
// q -> 1; the derivative is -60 q^3 (1 - q)^2 / r_max.
__device__ __forceinline__ float cutoff_val(float r, float rmax) {
  if (!(r < rmax)) return 0.f;
  const float q = r / rmax, t = 1.f - q;
  return t * t * t * (1.f + q * (3.f + q * (6.f + 10.f * q)));
}
__device__ __forceinline__ float cutoff_der(float r, float rmax) {
  if (!(r < rmax)) return 0.f;
  const float q = r / rmax, t = 1.f - q;
  return -60.f * q * q * q * t * t / rmax;
}

struct EdgeGeo {
  float vx, vy, vz, r, ux, uy, uz;
};

__device__ __forceinline__ EdgeGeo edge_geo(const float* pos, const int* send, const int* recv,
                                            const float* shift, int64_t e) {
  const int s = send[e], t = recv[e];
  EdgeGeo g;
  g.vx = pos[3 * t + 0] - pos[3 * s + 0];
  g.vy = pos[3 * t + 1] - pos[3 * s + 1];
  g.vz = pos[3 * t + 2] - pos[3 * s + 2];
  if (shift) {
    g.vx += shift[3 * e + 0];
    g.vy += shift[3 * e + 1];
    g.vz += shift[3 * e + 2];
  }
  g.r = sqrtf(g.vx * g.vx + g.vy * g.vy + g.vz * g.vz);
  const float inv = 1.f / fmaxf(g.r, 1e-12f);
  g.ux = g.vx * inv;
  g.uy = g.vy * inv;
  g.uz = g.vz * inv;
  return g;
}

// edge_feat[e, n*16 + m] = cut(r) rbf_n(r) Y_m(u), rbf_n = sqrt(2/rmax) sin(n pi r / rmax) / r
// (orb_geometry.py:65-97).  One thread per (edge, n); it writes 16 consecutive floats.
__global__ __launch_bounds__(256) void k_edge_features(const float* __restrict__ pos,
                                                       const int* __restrict__ send,
                                                       const int* __restrict__ recv,
                                                       const float* __restrict__ shift, float rmax,
                                                       int nb, float* __restrict__ vec,
                                                       float* __restrict__ feat,
                                                       float* __restrict__ cut, int64_t E) {
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= E * nb) return;
  const int64_t e = gid / nb;
  const int n = (int)(gid % nb);
  const EdgeGeo g = edge_geo(pos, send, recv, shift, e);
  float Y[16];
  sph_l3(g.ux, g.uy, g.uz, Y);
  const float w = (float)(n + 1) * (3.14159265358979323846f / rmax);
  const float rbf = sqrtf(2.f / rmax) * sinf(w * g.r) / g.r;
  const float c = cutoff_val(g.r, rmax);
  const float cr = c * rbf;
  floatx4* out = reinterpret_cast<floatx4*>(feat + (e * nb + n) * 16);
#pragma unroll
  for (int q = 0; q < 4; ++q)
    out[q] = floatx4{cr * Y[4 * q], cr * Y[4 * q + 1], cr * Y[4 * q + 2], cr * Y[4 * q + 3]};
  if (n == 0) {
    vec[3 * e + 0] = g.vx;
    vec[3 * e + 1] = g.vy;
    vec[3 * e + 2] = g.vz;
    cut[e] = c;
  }
}

// Closed-form VJP (orb_geometry.py:100-139): from g_feat [E, nb*16] and g_cut [E] to g_vec [E,3].
// The nb threads of an edge (a power-of-two group of consecutive lanes) each reduce one rbf row
// and combine the 16 angular partials with butterfly shuffles.
__global__ __launch_bounds__(256) void k_edge_features_bwd(const float* __restrict__ vec,
                                                           const float* __restrict__ g_feat,
                                                           const float* __restrict__ g_cut,
                                                           float rmax, int nb,
                                                           float* __restrict__ g_vec, int64_t E) {
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const bool live = gid < E * nb;
  const int64_t e = live ? gid / nb : 0;
  const int n = (int)(gid % nb);
  const float vx = vec[3 * e], vy = vec[3 * e + 1], vz = vec[3 * e + 2];
  const float r = sqrtf(vx * vx + vy * vy + vz * vz);
  const float ux = vx / r, uy = vy / r, uz = vz / r;
  float Y[16];
  sph_l3(ux, uy, uz, Y);
  const float w = (float)(n + 1) * (3.14159265358979323846f / rmax);
  const float pre = sqrtf(2.f / rmax);
  float sn, cs;
  sincosf(w * r, &sn, &cs);
  const float rbf = pre * sn / r;
  const float drbf = pre * (w * cs * r - sn) / (r * r);
  const float c = cutoff_val(r, rmax);
  float Q[16];
  float P = 0.f;
  const floatx4* gr = reinterpret_cast<const floatx4*>(g_feat + (e * nb + n) * 16);
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const floatx4 v = gr[q];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      P += v[k] * Y[4 * q + k];
      Q[4 * q + k] = v[k] * rbf;
    }
  }
  float S = rbf * P;            // this row's share of sum_{n,m} g rbf Y
  float GR = c * P * drbf;      // g_rbf[n] * d rbf_n / dr
  for (int o = 1; o < nb; o <<= 1) {
    S += __shfl_xor(S, o, 64);
    GR += __shfl_xor(GR, o, 64);
#pragma unroll
    for (int m = 0; m < 16; ++m) Q[m] += __shfl_xor(Q[m], o, 64);
  }
  if (!live || n != 0) return;
  float gY[16];
#pragma unroll
  for (int m = 0; m < 16; ++m) gY[m] = c * Q[m];
  const float gc = g_cut[e] + S;
  const float gr_tot = GR + gc * cutoff_der(r, rmax);
  float gx, gy, gz;
  sph_l3_vjp(ux, uy, uz, gY, gx, gy, gz);
  const float rad = gx * ux + gy * uy + gz * uz;
  g_vec[3 * e + 0] = ux * gr_tot + (gx - ux * rad) / r;
  g_vec[3 * e + 1] = uy * gr_tot + (gy - uy * rad) / r;
  g_vec[3 * e + 2] = uz * gr_tot + (gz - uz * rad) / r;
}

// ------------------------------------------------------------------------------ row kernels
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

constexpr int kMaxQ = 4;  // row width up to 64 lanes x 4 x kMaxQ = 1024 floats
constexpr int kU = 4;     // edge rows in flight per lane in the segment sums

// y = h * rsqrt(mean(h^2) + eps) * w (RMSNorm, orb_model.py:92-112); u = y; x_new = x_old + y
// (residual, orb_model.py:266); optionally the next layer's attention gates on x_new:
// sig[r] = (sigmoid(x_new . w_r + b_r), sigmoid(x_new . w_s + b_s)) (orb_model.py:239-246).
// One wavefront per row.
__global__ __launch_bounds__(256) void k_rms_residual(
    const float* __restrict__ h, const float* __restrict__ w, const float* __restrict__ x_old,
    float* __restrict__ u, float* __restrict__ x_new, float* __restrict__ inv_out,
    const float* __restrict__ attn_w, const float* __restrict__ attn_b, float* __restrict__ sig,
    int64_t R, int C, float eps) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= R) return;
  const int nq = C / 4;
  const floatx4* hr = reinterpret_cast<const floatx4*>(h + row * C);
  floatx4 hv[kMaxQ];
  float ss = 0.f;
#pragma unroll
  for (int k = 0; k < kMaxQ; ++k) {
    const int q = lane + 64 * k;
    hv[k] = q < nq ? hr[q] : floatx4{0.f, 0.f, 0.f, 0.f};
    ss += hv[k][0] * hv[k][0] + hv[k][1] * hv[k][1] + hv[k][2] * hv[k][2] + hv[k][3] * hv[k][3];
  }
  ss = wave_sum(ss);
  const float inv = 1.f / sqrtf(ss / (float)C + eps);
  if (lane == 0 && inv_out) inv_out[row] = inv;
  float dr = 0.f, ds = 0.f;
#pragma unroll
  for (int k = 0; k < kMaxQ; ++k) {
    const int q = lane + 64 * k;
    if (q >= nq) continue;
    const floatx4 wv = reinterpret_cast<const floatx4*>(w)[q];
    floatx4 y = (hv[k] * inv) * wv;
    if (u) reinterpret_cast<floatx4*>(u + row * C)[q] = y;
    if (x_old) y += reinterpret_cast<const floatx4*>(x_old + row * C)[q];
    if (x_new) reinterpret_cast<floatx4*>(x_new + row * C)[q] = y;
    if (attn_w) {
      const floatx4 wr = reinterpret_cast<const floatx4*>(attn_w)[q];
      const floatx4 ws = reinterpret_cast<const floatx4*>(attn_w + C)[q];
      dr += y[0] * wr[0] + y[1] * wr[1] + y[2] * wr[2] + y[3] * wr[3];
      ds += y[0] * ws[0] + y[1] * ws[1] + y[2] * ws[2] + y[3] * ws[3];
    }
  }
  if (attn_w) {
    dr = wave_sum(dr);
    ds = wave_sum(ds);
    if (lane == 0) {
      sig[2 * row + 0] = tta_sigmoid_acc(dr + attn_b[0]);
      sig[2 * row + 1] = tta_sigmoid_acc(ds + attn_b[1]);
    }
  }
}

// RMSNorm VJP (orb_forces.py:67-79): g_h = inv w g - inv^3 / C * h * sum(g w h).
__global__ __launch_bounds__(256) void k_rms_bwd(const float* __restrict__ g,
                                                 const float* __restrict__ h,
                                                 const float* __restrict__ w,
                                                 const float* __restrict__ inv_in,
                                                 float* __restrict__ g_h, int64_t R, int C) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= R) return;
  const int nq = C / 4;
  floatx4 gw[kMaxQ], hv[kMaxQ];
  float s = 0.f;
#pragma unroll
  for (int k = 0; k < kMaxQ; ++k) {
    const int q = lane + 64 * k;
    gw[k] = hv[k] = floatx4{0.f, 0.f, 0.f, 0.f};
    if (q < nq) {
      gw[k] = reinterpret_cast<const floatx4*>(g + row * C)[q] *
              reinterpret_cast<const floatx4*>(w)[q];
      hv[k] = reinterpret_cast<const floatx4*>(h + row * C)[q];
    }
    s += gw[k][0] * hv[k][0] + gw[k][1] * hv[k][1] + gw[k][2] * hv[k][2] + gw[k][3] * hv[k][3];
  }
  s = wave_sum(s);
  const float inv = inv_in[row];
  const float t2 = inv * inv * inv * (s / (float)C);
#pragma unroll
  for (int k = 0; k < kMaxQ; ++k) {
    const int q = lane + 64 * k;
    if (q < nq) reinterpret_cast<floatx4*>(g_h + row * C)[q] = gw[k] * inv - hv[k] * t2;
  }
}

// node_in[n] = [nodes[n] | sum_{recv(e)=n} ue[e] a_r[e] | sum_{send(e)=n} ue[e] a_s[e]] with
// a = sigmoid gate * cutoff (orb_model.py:245-259).  One wavefront per node; KQ float4 groups of
// a row per lane (rows of up to 256 KQ floats) and U = 16 / KQ edge rows in flight per lane.
template <int KQ>
__global__ __launch_bounds__(256) void k_segsum(const float* __restrict__ ue,
                                                const float* __restrict__ sig,
                                                const float* __restrict__ cut,
                                                const int* __restrict__ send_ptr,
                                                const int* __restrict__ recv_ptr,
                                                const int* __restrict__ recv_perm,
                                                const float* __restrict__ nodes,
                                                float* __restrict__ node_in, int64_t N, int C) {
  constexpr int U = 16 / KQ;
  const int lane = threadIdx.x & 63;
  const int64_t n = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (n >= N) return;
  const int nq = C / 4;
  floatx4 sr[KQ], ssn[KQ];
#pragma unroll
  for (int k = 0; k < KQ; ++k) sr[k] = ssn[k] = floatx4{0.f, 0.f, 0.f, 0.f};
  // Up to 64 edges of a segment at a time: lane i fetches edge i's index and weight (one load
  // each for the wave), then the rows of U edges at a time are all in flight before any is added;
  // the additions keep the plain loop's edge order.
  const int r0 = recv_ptr[n], r1 = recv_ptr[n + 1];
  for (int j0 = r0; j0 < r1; j0 += 64) {
    const int cnt = min(64, r1 - j0);
    const int my_e = lane < cnt ? recv_perm[j0 + lane] : 0;
    const float my_w = lane < cnt ? sig[2 * my_e + 0] * cut[my_e] : 0.f;
    for (int u0 = 0; u0 < cnt; u0 += U) {
      // every row load is issued (past the chunk: its last edge again; past the row: its last
      // float4), so the compiler's wait counts stay exact; the extra values are not added
      floatx4 v[U][KQ];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int e = __shfl(my_e, min(u0 + u, cnt - 1), 64);
#pragma unroll
        for (int k = 0; k < KQ; ++k) {
          const int q = min(lane + 64 * k, nq - 1);
          v[u][k] = reinterpret_cast<const floatx4*>(ue + (int64_t)e * C)[q];
        }
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const float w = __shfl(my_w, u0 + u, 64);
        if (u0 + u < cnt)
#pragma unroll
          for (int k = 0; k < KQ; ++k) sr[k] += v[u][k] * w;
      }
    }
  }
  const int s0 = send_ptr[n], s1 = send_ptr[n + 1];
  for (int j0 = s0; j0 < s1; j0 += 64) {
    const int cnt = min(64, s1 - j0);
    const float my_w = lane < cnt ? sig[2 * (j0 + lane) + 1] * cut[j0 + lane] : 0.f;
    for (int u0 = 0; u0 < cnt; u0 += U) {
      floatx4 v[U][KQ];
#pragma unroll
      for (int u = 0; u < U; ++u)
#pragma unroll
        for (int k = 0; k < KQ; ++k) {
          const int q = min(lane + 64 * k, nq - 1);
          v[u][k] = reinterpret_cast<const floatx4*>(
              ue + (int64_t)(j0 + min(u0 + u, cnt - 1)) * C)[q];
        }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const float w = __shfl(my_w, u0 + u, 64);
        if (u0 + u < cnt)
#pragma unroll
          for (int k = 0; k < KQ; ++k) ssn[k] += v[u][k] * w;
      }
    }
  }
  floatx4* out = reinterpret_cast<floatx4*>(node_in + n * 3 * C);
#pragma unroll
  for (int k = 0; k < KQ; ++k) {
    const int q = lane + 64 * k;
    if (q >= nq) continue;
    out[q] = reinterpret_cast<const floatx4*>(nodes + n * C)[q];
    out[nq + q] = sr[k];
    out[2 * nq + q] = ssn[k];
  }
}

// Per-edge backward of one interaction layer's edge side (orb_forces.py:107-147):
//   g_ue   = g_e + g_recv_agg[recv] a_r + g_sent_agg[send] a_s      (scatter adjoint = gather)
//   g_a_r  = <g_recv_agg[recv], ue>, g_a_s = <g_sent_agg[send], ue>
//   g_h2   = RMSNorm VJP of g_ue                                       (written)
//   g_cut += g_a_r sig_r + g_a_s sig_s                                 (accumulated over layers)
//   g_e   += sig'(.) cut g_a_r w_r + sig'(.) cut g_a_s w_s             (attention adjoint, in place)
// g_node_in rows are [g_nodes_direct | g_recv_agg | g_sent_agg] (stride 3C).
__global__ __launch_bounds__(256) void k_edge_bwd(
    float* __restrict__ g_e, const float* __restrict__ g_node_in, const float* __restrict__ ue,
    const float* __restrict__ sig, const float* __restrict__ cut, const float* __restrict__ h2,
    const float* __restrict__ inv_in, const float* __restrict__ wn,
    const float* __restrict__ attn_w, const int* __restrict__ send, const int* __restrict__ recv,
    float* __restrict__ g_h2, float* __restrict__ g_cut, int64_t E, int C) {
  const int lane = threadIdx.x & 63;
  const int64_t e = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (e >= E) return;
  const int nq = C / 4;
  const float sr = sig[2 * e], ss = sig[2 * e + 1], c = cut[e];
  const float ar = sr * c, as = ss * c;
  const floatx4* gR = reinterpret_cast<const floatx4*>(g_node_in + (int64_t)recv[e] * 3 * C) + nq;
  const floatx4* gS =
      reinterpret_cast<const floatx4*>(g_node_in + (int64_t)send[e] * 3 * C) + 2 * nq;
  floatx4 gu[kMaxQ], ge[kMaxQ], hv[kMaxQ];
  float dr = 0.f, ds = 0.f, sd = 0.f;
#pragma unroll
  for (int k = 0; k < kMaxQ; ++k) {
    const int q = lane + 64 * k;
    gu[k] = ge[k] = hv[k] = floatx4{0.f, 0.f, 0.f, 0.f};
    if (q >= nq) continue;
    const floatx4 r4 = gR[q], s4 = gS[q];
    const floatx4 u4 = reinterpret_cast<const floatx4*>(ue + e * C)[q];
    ge[k] = reinterpret_cast<const floatx4*>(g_e + e * C)[q];
    hv[k] = reinterpret_cast<const floatx4*>(h2 + e * C)[q];
    const floatx4 w4 = reinterpret_cast<const floatx4*>(wn)[q];
    gu[k] = (ge[k] + r4 * ar + s4 * as) * w4;  // g_ue * w
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      dr += r4[i] * u4[i];
      ds += s4[i] * u4[i];
      sd += gu[k][i] * hv[k][i];
    }
  }
  dr = wave_sum(dr);
  ds = wave_sum(ds);
  sd = wave_sum(sd);
  const float inv = inv_in[e];
  const float t2 = inv * inv * inv * (sd / (float)C);
  const float glr = dr * c * sr * (1.f - sr);
  const float gls = ds * c * ss * (1.f - ss);
#pragma unroll
  for (int k = 0; k < kMaxQ; ++k) {
    const int q = lane + 64 * k;
    if (q >= nq) continue;
    reinterpret_cast<floatx4*>(g_h2 + e * C)[q] = gu[k] * inv - hv[k] * t2;
    const floatx4 wr = reinterpret_cast<const floatx4*>(attn_w)[q];
    const floatx4 ws = reinterpret_cast<const floatx4*>(attn_w + C)[q];
    reinterpret_cast<floatx4*>(g_e + e * C)[q] = ge[k] + wr * glr + ws * gls;
  }
  if (lane == 0) g_cut[e] += dr * sr + ds * ss;
}

// out[n] = [sum_{send(e)=n} x[e] | sum_{recv(e)=n} x[e]], x [E, H]; one wavefront per node,
// 256-float chunks.  The node-level adjoint of the first edge-MLP layer's gathered inputs.
__global__ __launch_bounds__(256) void k_node_segsum2(const float* __restrict__ x,
                                                      const int* __restrict__ send_ptr,
                                                      const int* __restrict__ recv_ptr,
                                                      const int* __restrict__ recv_perm,
                                                      float* __restrict__ out, int64_t N, int H) {
  const int lane = threadIdx.x & 63;
  const int64_t n = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (n >= N) return;
  const int nq = H / 4;
  floatx4* o = reinterpret_cast<floatx4*>(out + n * 2 * H);
  const int s0 = send_ptr[n], s1 = send_ptr[n + 1], r0 = recv_ptr[n], r1 = recv_ptr[n + 1];
  // Column blocks of 64 lanes x kMaxQ float4; within a block, edges in groups of kU whose rows
  // are all loaded before the (edge-ordered) additions.
  for (int qb = 0; qb < nq; qb += 64 * kMaxQ) {
    floatx4 a[kMaxQ], b[kMaxQ];
#pragma unroll
    for (int k = 0; k < kMaxQ; ++k) a[k] = b[k] = floatx4{0.f, 0.f, 0.f, 0.f};
    for (int e0 = s0; e0 < s1; e0 += kU) {
      floatx4 v[kU][kMaxQ];
#pragma unroll
      for (int u = 0; u < kU; ++u)
#pragma unroll
        for (int k = 0; k < kMaxQ; ++k) {
          const int q = qb + lane + 64 * k;
          v[u][k] = (e0 + u < s1 && q < nq)
                        ? reinterpret_cast<const floatx4*>(x + (int64_t)(e0 + u) * H)[q]
                        : floatx4{0.f, 0.f, 0.f, 0.f};
        }
#pragma unroll
      for (int u = 0; u < kU; ++u)
        if (e0 + u < s1)
#pragma unroll
          for (int k = 0; k < kMaxQ; ++k) a[k] += v[u][k];
    }
    for (int j0 = r0; j0 < r1; j0 += 64) {
      const int cnt = min(64, r1 - j0);
      const int my_e = lane < cnt ? recv_perm[j0 + lane] : 0;
      for (int u0 = 0; u0 < cnt; u0 += kU) {
        floatx4 v[kU][kMaxQ];
#pragma unroll
        for (int u = 0; u < kU; ++u) {
          const int e = __shfl(my_e, u0 + u, 64);
#pragma unroll
          for (int k = 0; k < kMaxQ; ++k) {
            const int q = qb + lane + 64 * k;
            v[u][k] = (u0 + u < cnt && q < nq)
                          ? reinterpret_cast<const floatx4*>(x + (int64_t)e * H)[q]
                          : floatx4{0.f, 0.f, 0.f, 0.f};
          }
        }
#pragma unroll
        for (int u = 0; u < kU; ++u)
          if (u0 + u < cnt)
#pragma unroll
            for (int k = 0; k < kMaxQ; ++k) b[k] += v[u][k];
      }
    }
#pragma unroll
    for (int k = 0; k < kMaxQ; ++k) {
      const int q = qb + lane + 64 * k;
      if (q >= nq) continue;
      o[q] = a[k];
      o[nq + q] = b[k];
    }
  }
}

// Per-system mean over contiguous node ranges [ptr[k], ptr[k+1]) (orb_model.py:340-355).
__global__ __launch_bounds__(256) void k_segment_mean(const float* __restrict__ x,
                                                      const int* __restrict__ ptr,
                                                      float* __restrict__ out, int64_t K, int C) {
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= K * C) return;
  const int64_t k = gid / C;
  const int c = (int)(gid % C);
  float s = 0.f;
  for (int n = ptr[k]; n < ptr[k + 1]; ++n) s += x[(int64_t)n * C + c];
  out[gid] = s / (float)(ptr[k + 1] - ptr[k]);
}

// out[n] = g[batch[n]] / count(batch[n]) -- the mean's adjoint (orb_forces.py:207-229).
__global__ __launch_bounds__(256) void k_segment_mean_bwd(const float* __restrict__ g,
                                                          const int* __restrict__ batch,
                                                          const int* __restrict__ ptr,
                                                          float* __restrict__ out, int64_t N,
                                                          int C) {
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= N * C) return;
  const int64_t n = gid / C;
  const int c = (int)(gid % C);
  const int k = batch[n];
  out[gid] = g[(int64_t)k * C + c] / (float)(ptr[k + 1] - ptr[k]);
}

// out[n, :] = x[n, :] - mean of x over n's system (ForceHead net-force removal,
// orb_model.py:387-388, per system as in the batched form 401-404).  One wavefront per system:
// lane j sums rows j, j + 64, ... in order, then a fixed butterfly over the lanes, so the result
// does not depend on scheduling.  C <= kCenterMaxC columns.
constexpr int kCenterMaxC = 16;
// x and out are not __restrict__: the entry point allows out == x.
__global__ __launch_bounds__(256) void k_segment_center(const float* x,
                                                        const int* __restrict__ ptr, float* out,
                                                        int64_t K, int C) {
  const int lane = threadIdx.x & 63;
  const int64_t k = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (k >= K) return;
  const int n0 = ptr[k], n1 = ptr[k + 1];
  float acc[kCenterMaxC];
#pragma unroll
  for (int c = 0; c < kCenterMaxC; ++c) acc[c] = 0.f;
  for (int n = n0 + lane; n < n1; n += 64) {
#pragma unroll
    for (int c = 0; c < kCenterMaxC; ++c)
      if (c < C) acc[c] += x[(int64_t)n * C + c];
  }
  const float inv_cnt = 1.f / (float)max(n1 - n0, 1);
#pragma unroll
  for (int c = 0; c < kCenterMaxC; ++c)
    if (c < C) acc[c] = wave_sum(acc[c]) * inv_cnt;
  for (int n = n0 + lane; n < n1; n += 64) {
#pragma unroll
    for (int c = 0; c < kCenterMaxC; ++c)
      if (c < C) out[(int64_t)n * C + c] = x[(int64_t)n * C + c] - acc[c];
  }
}

// y[r, :C] += x[r, :C] with row strides ldx, ldy.
__global__ __launch_bounds__(256) void k_add_rows(const float* __restrict__ x, int64_t ldx,
                                                  float* __restrict__ y, int64_t ldy, int64_t R,
                                                  int C) {
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= R * C) return;
  const int64_t r = gid / C;
  const int c = (int)(gid % C);
  y[r * ldy + c] += x[r * ldx + c];
}

bool row_width_ok(int64_t C) { return C > 0 && C % 4 == 0 && C <= 256 * kMaxQ; }

}  // namespace

extern "C" int tta_orb_edge_features(const float* pos, const int* send, const int* recv,
                                     const float* shift, float r_max, int64_t nb, float* vec,
                                     float* feat, float* cut, int64_t N, int64_t E,
                                     hipStream_t stream) {
  TTA_CHECK_ARG(E >= 0 && N >= 0 && nb >= 1 && nb <= 64, "tta_orb_edge_features: bad sizes");
  TTA_CHECK_ARG(r_max > 0.f, "tta_orb_edge_features: r_max must be positive");
  if (E == 0) return tta::kOk;
  TTA_CHECK_ARG(pos && send && recv && vec && feat && cut, "tta_orb_edge_features: null pointer");
  hipLaunchKernelGGL(k_edge_features, dim3(tta_blocks(E * nb, 256)), dim3(256), 0, stream, pos,
                     send, recv, shift, r_max, (int)nb, vec, feat, cut, E);
  TTA_CHECK_LAUNCH("tta_orb_edge_features");
  return tta::kOk;
}

extern "C" int tta_orb_edge_features_bwd(const float* vec, const float* g_feat,
                                         const float* g_cut, float r_max, int64_t nb,
                                         float* g_vec, int64_t E, hipStream_t stream) {
  TTA_CHECK_ARG(E >= 0 && nb >= 1 && nb <= 64 && (nb & (nb - 1)) == 0,
                "tta_orb_edge_features_bwd: nb must be a power of two <= 64");
  if (E == 0) return tta::kOk;
  TTA_CHECK_ARG(vec && g_feat && g_cut && g_vec, "tta_orb_edge_features_bwd: null pointer");
  hipLaunchKernelGGL(k_edge_features_bwd, dim3(tta_blocks(E * nb, 256)), dim3(256), 0, stream,
                     vec, g_feat, g_cut, r_max, (int)nb, g_vec, E);
  TTA_CHECK_LAUNCH("tta_orb_edge_features_bwd");
  return tta::kOk;
}

extern "C" int tta_rms_residual(const float* h, const float* w, const float* x_old, float* u,
                                float* x_new, float* inv, const float* attn_w,
                                const float* attn_b, float* sig, int64_t R, int64_t C, float eps,
                                hipStream_t stream) {
  TTA_CHECK_ARG(R >= 0 && row_width_ok(C), "tta_rms_residual: C must be a multiple of 4, <= 1024");
  TTA_CHECK_ARG(!attn_w || (attn_b && sig), "tta_rms_residual: attention needs bias and output");
  if (R == 0) return tta::kOk;
  TTA_CHECK_ARG(h && w, "tta_rms_residual: null pointer");
  hipLaunchKernelGGL(k_rms_residual, dim3(tta_blocks(R, 4)), dim3(256), 0, stream, h, w, x_old, u,
                     x_new, inv, attn_w, attn_b, sig, R, (int)C, eps);
  TTA_CHECK_LAUNCH("tta_rms_residual");
  return tta::kOk;
}

extern "C" int tta_rms_bwd(const float* g, const float* h, const float* w, const float* inv,
                           float* g_h, int64_t R, int64_t C, hipStream_t stream) {
  TTA_CHECK_ARG(R >= 0 && row_width_ok(C), "tta_rms_bwd: C must be a multiple of 4, <= 1024");
  if (R == 0) return tta::kOk;
  TTA_CHECK_ARG(g && h && w && inv && g_h, "tta_rms_bwd: null pointer");
  hipLaunchKernelGGL(k_rms_bwd, dim3(tta_blocks(R, 4)), dim3(256), 0, stream, g, h, w, inv, g_h,
                     R, (int)C);
  TTA_CHECK_LAUNCH("tta_rms_bwd");
  return tta::kOk;
}

extern "C" int tta_orb_segsum(const float* ue, const float* sig, const float* cut,
                              const int* send_ptr, const int* recv_ptr, const int* recv_perm,
                              const float* nodes, float* node_in, int64_t N, int64_t E, int64_t C,
                              hipStream_t stream) {
  TTA_CHECK_ARG(N >= 0 && E >= 0 && row_width_ok(C), "tta_orb_segsum: bad sizes");
  if (N == 0) return tta::kOk;
  TTA_CHECK_ARG(send_ptr && recv_ptr && nodes && node_in && (E == 0 || (ue && sig && cut && recv_perm)),
                "tta_orb_segsum: null pointer");
  // float4 groups per lane: rows of up to 256, 512, 768 or 1024 floats
  const int kq = (int)((C / 4 + 63) / 64);
  auto launch = [&](auto kern) {
    hipLaunchKernelGGL(kern, dim3(tta_blocks(N, 4)), dim3(256), 0, stream, ue, sig, cut,
                       send_ptr, recv_ptr, recv_perm, nodes, node_in, N, (int)C);
  };
  if (kq <= 1)
    launch(k_segsum<1>);
  else if (kq == 2)
    launch(k_segsum<2>);
  else
    launch(k_segsum<4>);
  TTA_CHECK_LAUNCH("tta_orb_segsum");
  return tta::kOk;
}

extern "C" int tta_orb_edge_bwd(float* g_e, const float* g_node_in, const float* ue,
                                const float* sig, const float* cut, const float* h2,
                                const float* inv, const float* wn, const float* attn_w,
                                const int* send, const int* recv, float* g_h2, float* g_cut,
                                int64_t N, int64_t E, int64_t C, hipStream_t stream) {
  TTA_CHECK_ARG(N >= 0 && E >= 0 && row_width_ok(C), "tta_orb_edge_bwd: bad sizes");
  if (E == 0) return tta::kOk;
  TTA_CHECK_ARG(g_e && g_node_in && ue && sig && cut && h2 && inv && wn && attn_w && send &&
                    recv && g_h2 && g_cut,
                "tta_orb_edge_bwd: null pointer");
  hipLaunchKernelGGL(k_edge_bwd, dim3(tta_blocks(E, 4)), dim3(256), 0, stream, g_e, g_node_in, ue,
                     sig, cut, h2, inv, wn, attn_w, send, recv, g_h2, g_cut, E, (int)C);
  TTA_CHECK_LAUNCH("tta_orb_edge_bwd");
  return tta::kOk;
}

extern "C" int tta_orb_node_segsum2(const float* x, const int* send_ptr, const int* recv_ptr,
                                    const int* recv_perm, float* out, int64_t N, int64_t E,
                                    int64_t H, hipStream_t stream) {
  TTA_CHECK_ARG(N >= 0 && E >= 0 && H > 0 && H % 4 == 0, "tta_orb_node_segsum2: bad sizes");
  if (N == 0) return tta::kOk;
  TTA_CHECK_ARG(send_ptr && recv_ptr && out && (E == 0 || (x && recv_perm)),
                "tta_orb_node_segsum2: null pointer");
  hipLaunchKernelGGL(k_node_segsum2, dim3(tta_blocks(N, 4)), dim3(256), 0, stream, x, send_ptr,
                     recv_ptr, recv_perm, out, N, (int)H);
  TTA_CHECK_LAUNCH("tta_orb_node_segsum2");
  return tta::kOk;
}

extern "C" int tta_segment_mean(const float* x, const int* ptr, float* out, int64_t K, int64_t C,
                                hipStream_t stream) {
  TTA_CHECK_ARG(K >= 0 && C > 0, "tta_segment_mean: bad sizes");
  if (K == 0) return tta::kOk;
  TTA_CHECK_ARG(x && ptr && out, "tta_segment_mean: null pointer");
  hipLaunchKernelGGL(k_segment_mean, dim3(tta_blocks(K * C, 256)), dim3(256), 0, stream, x, ptr,
                     out, K, (int)C);
  TTA_CHECK_LAUNCH("tta_segment_mean");
  return tta::kOk;
}

extern "C" int tta_segment_mean_bwd(const float* g, const int* batch, const int* ptr, float* out,
                                    int64_t N, int64_t C, hipStream_t stream) {
  TTA_CHECK_ARG(N >= 0 && C > 0, "tta_segment_mean_bwd: bad sizes");
  if (N == 0) return tta::kOk;
  TTA_CHECK_ARG(g && batch && ptr && out, "tta_segment_mean_bwd: null pointer");
  hipLaunchKernelGGL(k_segment_mean_bwd, dim3(tta_blocks(N * C, 256)), dim3(256), 0, stream, g,
                     batch, ptr, out, N, (int)C);
  TTA_CHECK_LAUNCH("tta_segment_mean_bwd");
  return tta::kOk;
}

extern "C" int tta_segment_center(const float* x, const int* ptr, float* out, int64_t K,
                                  int64_t C, hipStream_t stream) {
  TTA_CHECK_ARG(K >= 0 && C > 0 && C <= kCenterMaxC,
                "tta_segment_center: bad sizes (1 <= C <= 16)");
  if (K == 0) return tta::kOk;
  TTA_CHECK_ARG(x && ptr && out, "tta_segment_center: null pointer");
  hipLaunchKernelGGL(k_segment_center, dim3((unsigned)((K + 3) / 4)), dim3(256), 0, stream, x, ptr,
                     out, K, (int)C);
  TTA_CHECK_LAUNCH("tta_segment_center");
  return tta::kOk;
}

extern "C" int tta_add_rows(const float* x, int64_t ldx, float* y, int64_t ldy, int64_t R,
                            int64_t C, hipStream_t stream) {
  TTA_CHECK_ARG(R >= 0 && C >= 0 && ldx >= C && ldy >= C, "tta_add_rows: bad sizes");
  if (R == 0 || C == 0) return tta::kOk;
  TTA_CHECK_ARG(x && y, "tta_add_rows: null pointer");
  hipLaunchKernelGGL(k_add_rows, dim3(tta_blocks(R * C, 256)), dim3(256), 0, stream, x, ldx, y,
                     ldy, R, (int)C);
  TTA_CHECK_LAUNCH("tta_add_rows");
  return tta::kOk;
}
