// Edge-frame rotation kernels of the eSCN-MD message block (lmax = mmax = 2, 9 coefficients).
//
// The per-edge Wigner matrix W[e] (m-primed rows x natural-order columns) is block diagonal by
// degree, so it is carried as 35 packed coefficients in the reference's pack order
// (tt_atom/rotation.py:196-208, row-major over (m, j)):
//   m=0: j=0 | m=1: j=1..3 | m=2: j=4..8 | m=3: j=1..3 | m=4: j=4..8 | m=5: j=1..3 |
//   m=6: j=4..8 | m=7: j=4..8 | m=8: j=4..8                              (offsets 0,1,4,9,...,30)
// The inverse rotation is W^T (geometry.py:211), so one coefficient array serves both
// directions.  Edge tensors are flat [E, 9, W] coefficient-major, W channels per coefficient.
//
// Work mapping: each edge (or node, for the segmented reductions) is owned by a group of G lanes
// (G = min(64, W/4)); a lane handles QPL float4 channel quads.  Channel reductions (coefficient
// adjoints, envelope adjoint) are butterfly sums inside the lane group, so every output is
// written by exactly one lane with plain stores: no float atomics, deterministic results.
#include "common.h"

typedef float floatx4 __attribute__((ext_vector_type(4)));

namespace {

constexpr int NSPH = 9;
constexpr int NNZ = 35;

__device__ __forceinline__ floatx4 ld4(const float* p) { return *reinterpret_cast<const floatx4*>(p); }
__device__ __forceinline__ void st4(float* p, floatx4 v) { *reinterpret_cast<floatx4*>(p) = v; }
__device__ __forceinline__ floatx4 z4() { return floatx4{0.f, 0.f, 0.f, 0.f}; }
__device__ __forceinline__ float dot4(floatx4 a, floatx4 b) {
  return a[0] * b[0] + a[1] * b[1] + a[2] * b[2] + a[3] * b[3];
}

// out[m] = sum_j W[m, j] in[j]   (node SH -> edge frame; also the adjoint of the inverse rotation)
__device__ __forceinline__ void rot_fwd(const float* c, const floatx4* in, floatx4* out) {
  out[0] = c[0] * in[0];
  const int m1[3] = {1, 3, 5}, k1[3] = {1, 9, 17};
#pragma unroll
  for (int r = 0; r < 3; ++r) {
    const int k = k1[r];
    out[m1[r]] = c[k] * in[1] + c[k + 1] * in[2] + c[k + 2] * in[3];
  }
  const int m2[5] = {2, 4, 6, 7, 8}, k2[5] = {4, 12, 20, 25, 30};
#pragma unroll
  for (int r = 0; r < 5; ++r) {
    const int k = k2[r];
    out[m2[r]] = c[k] * in[4] + c[k + 1] * in[5] + c[k + 2] * in[6] + c[k + 3] * in[7] +
                 c[k + 4] * in[8];
  }
}

// out[j] = sum_m W[m, j] in[m]   (edge frame -> node SH; also the adjoint of the forward rotation)
// Only the first NIN m-primed inputs are non-zero (NIN = 3: the m = 0 block alone).
template <int NIN>
__device__ __forceinline__ void rot_inv(const float* c, const floatx4* in, floatx4* out) {
  out[0] = c[0] * in[0];
#pragma unroll
  for (int q = 0; q < 3; ++q) {
    floatx4 v = c[1 + q] * in[1];
    if (NIN > 3) v = v + c[9 + q] * in[3] + c[17 + q] * in[5];
    out[1 + q] = v;
  }
#pragma unroll
  for (int q = 0; q < 5; ++q) {
    floatx4 v = c[4 + q] * in[2];
    if (NIN > 3) v = v + c[12 + q] * in[4] + c[20 + q] * in[6] + c[25 + q] * in[7] + c[30 + q] * in[8];
    out[4 + q] = v;
  }
}

// Coefficient adjoint partials: gc[k] += <a[m_k], b[j_k]> over one channel quad, where a is the
// m-primed-side tensor and b the natural-side tensor.  Only k with m_k < NIN when NIN = 3.
template <int NIN>
__device__ __forceinline__ void coef_partials(const floatx4* a, const floatx4* b, float* gc) {
  gc[0] += dot4(a[0], b[0]);
  const int m1[3] = {1, 3, 5}, k1[3] = {1, 9, 17};
#pragma unroll
  for (int r = 0; r < 3; ++r) {
    if (m1[r] >= NIN) continue;
#pragma unroll
    for (int q = 0; q < 3; ++q) gc[k1[r] + q] += dot4(a[m1[r]], b[1 + q]);
  }
  const int m2[5] = {2, 4, 6, 7, 8}, k2[5] = {4, 12, 20, 25, 30};
#pragma unroll
  for (int r = 0; r < 5; ++r) {
    if (m2[r] >= NIN) continue;
#pragma unroll
    for (int q = 0; q < 5; ++q) gc[k2[r] + q] += dot4(a[m2[r]], b[4 + q]);
  }
}

// Radial block of each m-primed coefficient: m0 {0,1,2} own blocks 0..2; the m=+-1 real/imag
// pairs (3,5) and (4,6) share blocks 3 and 4; the m=+-2 pair (7,8) shares block 5
// (so2.py:197-209: the radial output is duplicated as [m0 | m1 | m1 | m2 | m2]).
__device__ __forceinline__ int rad_block(int m) {
  const int rb[9] = {0, 1, 2, 3, 4, 3, 4, 5, 5};
  return rb[m];
}

struct Lanes {
  int G;    // lanes per item
  int QPL;  // channel quads per lane
};

static bool lanes_for(int64_t W, Lanes& l) {
  if (W <= 0 || W % 4) return false;
  const int64_t W4 = W / 4;
  if (W4 <= 64) {
    if (W4 & (W4 - 1)) return false;  // power of two so groups tile a wave
    l.G = (int)W4;
    l.QPL = 1;
  } else {
    if (W4 % 64) return false;
    l.G = 64;
    l.QPL = (int)(W4 / 64);
  }
  return true;
}

__device__ __forceinline__ void load_coef(const float* coef, int64_t e, float* c) {
#pragma unroll
  for (int k = 0; k < NNZ; ++k) c[k] = coef[e * NNZ + k];
}

// -------------------------------------------------------------------------------------------
// Forward: out[e, m, :] = (sum_j W[e,m,j] [x[src_e, j, :] | x[tgt_e, j, :]]) * rad[e, rb(m), :]
// (edgewise.py:52-69 gather + interleave + rotate, so2.py:263-277 radial multiply).
template <bool RAD>
__global__ __launch_bounds__(256) void k_gather_rotate(const float* __restrict__ x,
                                                       const int* __restrict__ src,
                                                       const int* __restrict__ tgt,
                                                       const float* __restrict__ coef,
                                                       const float* __restrict__ rad,
                                                       float* __restrict__ out, int E, int C,
                                                       Lanes ln) {
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t e = gid / ln.G;
  const int gl = (int)(gid % ln.G);
  if (e >= E) return;
  const int W = 2 * C, C4 = C / 4;
  float c[NNZ];
  load_coef(coef, e, c);
  const int64_t s = src[e], t = tgt[e];
  for (int q = 0; q < ln.QPL; ++q) {
    const int qd = gl + q * ln.G;
    const float* row = qd < C4 ? x + s * NSPH * C + 4 * qd : x + t * NSPH * C + 4 * (qd - C4);
    floatx4 in[NSPH], o[NSPH];
#pragma unroll
    for (int j = 0; j < NSPH; ++j) in[j] = ld4(row + j * C);
    rot_fwd(c, in, o);
    float* orow = out + e * NSPH * W + 4 * qd;
#pragma unroll
    for (int m = 0; m < NSPH; ++m) {
      floatx4 v = o[m];
      if (RAD) v = v * ld4(rad + e * 6 * W + rad_block(m) * W + 4 * qd);
      st4(orow + m * W, v);
    }
  }
}

// -------------------------------------------------------------------------------------------
// Backward of k_gather_rotate.  Recomputes the gathered input and the rotation instead of
// storing them.  Writes g_mcat [E, 9, 2C] (adjoint of the interleaved gather, scattered to
// nodes by k_node_gather_sum), g_rad [E, 6, 2C] (adjoint at the radial output, duplicate blocks
// collapsed) and accumulates the coefficient adjoint g_coef[e, k] += <g_mrot[m_k], m_cat[j_k]>
// (rotation.py:225-260 semantics).
template <bool RAD>
__global__ __launch_bounds__(256) void k_gather_rotate_bw(
    const float* __restrict__ g_xf, const float* __restrict__ rad, const float* __restrict__ x,
    const int* __restrict__ src, const int* __restrict__ tgt, const float* __restrict__ coef,
    float* __restrict__ g_rad, float* __restrict__ g_mcat, float* __restrict__ g_coef, int E,
    int C, Lanes ln) {
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t e = gid / ln.G;
  const int gl = (int)(gid % ln.G);
  if (e >= E) return;  // whole lane groups exit together (G divides the block size)
  const int W = 2 * C, C4 = C / 4;
  float c[NNZ];
  load_coef(coef, e, c);
  float gc[NNZ];
#pragma unroll
  for (int k = 0; k < NNZ; ++k) gc[k] = 0.f;
  const int64_t s = src[e], t = tgt[e];
  for (int q = 0; q < ln.QPL; ++q) {
    const int qd = gl + q * ln.G;
    const float* row = qd < C4 ? x + s * NSPH * C + 4 * qd : x + t * NSPH * C + 4 * (qd - C4);
    floatx4 in[NSPH], gm[NSPH];
#pragma unroll
    for (int j = 0; j < NSPH; ++j) in[j] = ld4(row + j * C);
#pragma unroll
    for (int m = 0; m < NSPH; ++m) gm[m] = ld4(g_xf + e * NSPH * W + m * W + 4 * qd);
    if (RAD) {
      floatx4 mr[NSPH];
      rot_fwd(c, in, mr);
      floatx4 gr[6];
#pragma unroll
      for (int b = 0; b < 6; ++b) gr[b] = z4();
#pragma unroll
      for (int m = 0; m < NSPH; ++m) gr[rad_block(m)] = gr[rad_block(m)] + gm[m] * mr[m];
#pragma unroll
      for (int b = 0; b < 6; ++b) st4(g_rad + e * 6 * W + b * W + 4 * qd, gr[b]);
#pragma unroll
      for (int m = 0; m < NSPH; ++m) gm[m] = gm[m] * ld4(rad + e * 6 * W + rad_block(m) * W + 4 * qd);
    }
    floatx4 gi[NSPH];
    rot_inv<9>(c, gm, gi);
#pragma unroll
    for (int j = 0; j < NSPH; ++j) st4(g_mcat + e * NSPH * W + j * W + 4 * qd, gi[j]);
    coef_partials<9>(gm, in, gc);
  }
#pragma unroll
  for (int k = 0; k < NNZ; ++k) gc[k] = tta_group_sum(gc[k], ln.G);
  if (gl == 0) {
#pragma unroll
    for (int k = 0; k < NNZ; ++k) g_coef[e * NNZ + k] += gc[k];
  }
}

// -------------------------------------------------------------------------------------------
// Inverse rotation + envelope + destination-sorted segmented sum (+ residual):
//   out[n, j, :] = res[n, j, :] + sum_{e in [ptr[n], ptr[n+1])} contrib_e[j, :]
// ENV_FIRST (edgewise.py:72-86):  contrib = W^T (m[e] * env[e])
// otherwise (geometry.py:269-276, edge-degree init): contrib = ((W^T pad(m[e])) * env[e]) / div
// Edges of a segment are summed in ascending order starting from zero, then the residual is
// added: the order index_add_ followed by "+ x_res" uses.
template <int NIN, bool ENV_FIRST>
__global__ __launch_bounds__(256) void k_rotate_env_segsum(
    const float* __restrict__ m, const float* __restrict__ coef, const float* __restrict__ env,
    const int* __restrict__ ptr, const float* __restrict__ res, float* __restrict__ out, int N,
    int C, float div, Lanes ln) {
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t n = gid / ln.G;
  const int gl = (int)(gid % ln.G);
  if (n >= N) return;
  const int e0 = ptr[n], e1 = ptr[n + 1];
  for (int q = 0; q < ln.QPL; ++q) {
    const int qd = gl + q * ln.G;
    floatx4 acc[NSPH];
#pragma unroll
    for (int j = 0; j < NSPH; ++j) acc[j] = z4();
    for (int e = e0; e < e1; ++e) {
      float c[NNZ];
      load_coef(coef, e, c);
      const float ev = env[e];
      floatx4 in[NSPH], o[NSPH];
#pragma unroll
      for (int mm = 0; mm < NSPH; ++mm) {
        if (mm < NIN) {
          in[mm] = ld4(m + (int64_t)e * NIN * C + mm * C + 4 * qd);
          if (ENV_FIRST) in[mm] = in[mm] * ev;
        } else {
          in[mm] = z4();
        }
      }
      rot_inv<NIN>(c, in, o);
#pragma unroll
      for (int j = 0; j < NSPH; ++j) {
        floatx4 v = o[j];
        if (!ENV_FIRST) v = (v * ev) / div;
        acc[j] = acc[j] + v;
      }
    }
#pragma unroll
    for (int j = 0; j < NSPH; ++j) {
      floatx4 v = acc[j];
      if (res) v = v + ld4(res + n * NSPH * C + j * C + 4 * qd);
      st4(out + n * NSPH * C + j * C + 4 * qd, v);
    }
  }
}

// -------------------------------------------------------------------------------------------
// Backward of k_rotate_env_segsum for one edge (the scatter adjoint is a gather by tgt):
// ENV_FIRST (forces.py:366-376):
//   g_back = g_node[tgt]; g_env_in = W g_back; g_m = g_env_in * env;
//   g_env += <g_env_in, m>;  g_coef(m,j) += <g_back[j], m[m] * env>
// otherwise (edge-degree, forward v = ((W^T pad(m)) * env) / div):
//   g_v2 = g_node[tgt] / div; g_v1 = g_v2 * env; g_env += <g_v2, W^T pad(m)>;
//   g_m = (W g_v1)[:NIN];  g_coef(m,j) += <g_v1[j], pad(m)[m]>
template <int NIN, bool ENV_FIRST>
__global__ __launch_bounds__(256) void k_rotate_env_segsum_bw(
    const float* __restrict__ g_node, const int* __restrict__ tgt, const float* __restrict__ m,
    const float* __restrict__ coef, const float* __restrict__ env, float* __restrict__ g_m,
    float* __restrict__ g_coef, float* __restrict__ g_env, int E, int C, float div, Lanes ln) {
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t e = gid / ln.G;
  const int gl = (int)(gid % ln.G);
  if (e >= E) return;
  float c[NNZ];
  load_coef(coef, e, c);
  const float ev = env[e];
  const int64_t t = tgt[e];
  float gc[NNZ];
#pragma unroll
  for (int k = 0; k < NNZ; ++k) gc[k] = 0.f;
  float genv = 0.f;
  for (int q = 0; q < ln.QPL; ++q) {
    const int qd = gl + q * ln.G;
    floatx4 gb[NSPH], mi[NSPH];
#pragma unroll
    for (int j = 0; j < NSPH; ++j) gb[j] = ld4(g_node + t * NSPH * C + j * C + 4 * qd);
#pragma unroll
    for (int mm = 0; mm < NSPH; ++mm)
      mi[mm] = mm < NIN ? ld4(m + e * NIN * C + mm * C + 4 * qd) : z4();
    if (ENV_FIRST) {
      floatx4 gin[NSPH], me[NSPH];
      rot_fwd(c, gb, gin);
#pragma unroll
      for (int mm = 0; mm < NSPH; ++mm) {
        me[mm] = mi[mm] * ev;
        if (mm >= NIN) continue;
        genv += dot4(gin[mm], mi[mm]);
        st4(g_m + e * NIN * C + mm * C + 4 * qd, gin[mm] * ev);
      }
      coef_partials<NIN>(me, gb, gc);
    } else {
      floatx4 v1[NSPH], g1[NSPH], gin[NSPH];
      rot_inv<NIN>(c, mi, v1);
#pragma unroll
      for (int j = 0; j < NSPH; ++j) {
        const floatx4 g2 = gb[j] / div;
        genv += dot4(g2, v1[j]);
        g1[j] = g2 * ev;
      }
      rot_fwd(c, g1, gin);
#pragma unroll
      for (int mm = 0; mm < NIN; ++mm) st4(g_m + e * NIN * C + mm * C + 4 * qd, gin[mm]);
      coef_partials<NIN>(mi, g1, gc);
    }
  }
#pragma unroll
  for (int k = 0; k < NNZ; ++k) gc[k] = tta_group_sum(gc[k], ln.G);
  genv = tta_group_sum(genv, ln.G);
  if (gl == 0) {
#pragma unroll
    for (int k = 0; k < NNZ; ++k) g_coef[e * NNZ + k] += gc[k];
    g_env[e] += genv;
  }
}

// -------------------------------------------------------------------------------------------
// Node adjoint of the interleaved src|tgt gather (forces.py:384-412):
//   g_x[n] = sum_{edges with src = n} g_mcat[e, :, 0:C] + sum_{edges with tgt = n} g_mcat[e, :, C:2C]
// src edges come through a src-sorted permutation (src_ptr / src_perm), tgt edges are the
// contiguous destination segments.  Optional residual: out = (src sum + tgt sum) + res.
__global__ __launch_bounds__(256) void k_node_gather_sum(
    const float* __restrict__ g_mcat, const int* __restrict__ src_ptr,
    const int* __restrict__ src_perm, const int* __restrict__ tgt_ptr,
    const float* __restrict__ res, float* __restrict__ out, int N, int C, Lanes ln) {
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t n = gid / ln.G;
  const int gl = (int)(gid % ln.G);
  if (n >= N) return;
  const int W = 2 * C;
  for (int q = 0; q < ln.QPL; ++q) {
    const int qd = gl + q * ln.G;
    floatx4 a[NSPH], b[NSPH];
#pragma unroll
    for (int j = 0; j < NSPH; ++j) a[j] = b[j] = z4();
    for (int k = src_ptr[n]; k < src_ptr[n + 1]; ++k) {
      const int64_t e = src_perm[k];
#pragma unroll
      for (int j = 0; j < NSPH; ++j) a[j] = a[j] + ld4(g_mcat + e * NSPH * W + j * W + 4 * qd);
    }
    for (int64_t e = tgt_ptr[n]; e < tgt_ptr[n + 1]; ++e) {
#pragma unroll
      for (int j = 0; j < NSPH; ++j) b[j] = b[j] + ld4(g_mcat + e * NSPH * W + j * W + C + 4 * qd);
    }
#pragma unroll
    for (int j = 0; j < NSPH; ++j) {
      floatx4 v = a[j] + b[j];
      if (res) v = v + ld4(res + n * NSPH * C + j * C + 4 * qd);
      st4(out + n * NSPH * C + j * C + 4 * qd, v);
    }
  }
}

}  // namespace

// =========================================================================== C ABI
extern "C" int tta_gather_rotate(const float* x, const int* src, const int* tgt,
                                 const float* coef, const float* rad, float* out, int64_t N,
                                 int64_t E, int64_t C, hipStream_t stream) {
  Lanes ln;
  TTA_CHECK_ARG(C > 0 && C % 4 == 0 && lanes_for(2 * C, ln),
                "tta_gather_rotate: unsupported channel count C=%lld", (long long)C);
  TTA_CHECK_ARG(E >= 0 && N >= 0 && E < (1ll << 31), "tta_gather_rotate: bad sizes");
  if (E == 0) return tta::kOk;
  TTA_CHECK_ARG(x && src && tgt && coef && out, "tta_gather_rotate: null pointer");
  const unsigned blocks = tta_blocks(E * ln.G, 256);
  if (rad)
    hipLaunchKernelGGL(k_gather_rotate<true>, dim3(blocks), dim3(256), 0, stream, x, src, tgt,
                       coef, rad, out, (int)E, (int)C, ln);
  else
    hipLaunchKernelGGL(k_gather_rotate<false>, dim3(blocks), dim3(256), 0, stream, x, src, tgt,
                       coef, rad, out, (int)E, (int)C, ln);
  TTA_CHECK_LAUNCH("tta_gather_rotate");
  return tta::kOk;
}

extern "C" int tta_gather_rotate_bw(const float* g_xf, const float* rad, const float* x,
                                    const int* src, const int* tgt, const float* coef,
                                    float* g_rad, float* g_mcat, float* g_coef, int64_t N,
                                    int64_t E, int64_t C, hipStream_t stream) {
  Lanes ln;
  TTA_CHECK_ARG(C > 0 && C % 4 == 0 && lanes_for(2 * C, ln),
                "tta_gather_rotate_bw: unsupported channel count C=%lld", (long long)C);
  TTA_CHECK_ARG(E >= 0 && N >= 0 && E < (1ll << 31), "tta_gather_rotate_bw: bad sizes");
  if (E == 0) return tta::kOk;
  TTA_CHECK_ARG(g_xf && x && src && tgt && coef && g_mcat && g_coef,
                "tta_gather_rotate_bw: null pointer");
  TTA_CHECK_ARG(!rad == !g_rad, "tta_gather_rotate_bw: rad and g_rad must be given together");
  const unsigned blocks = tta_blocks(E * ln.G, 256);
  if (rad)
    hipLaunchKernelGGL(k_gather_rotate_bw<true>, dim3(blocks), dim3(256), 0, stream, g_xf, rad,
                       x, src, tgt, coef, g_rad, g_mcat, g_coef, (int)E, (int)C, ln);
  else
    hipLaunchKernelGGL(k_gather_rotate_bw<false>, dim3(blocks), dim3(256), 0, stream, g_xf, rad,
                       x, src, tgt, coef, g_rad, g_mcat, g_coef, (int)E, (int)C, ln);
  TTA_CHECK_LAUNCH("tta_gather_rotate_bw");
  return tta::kOk;
}

extern "C" int tta_rotate_env_segsum(const float* m, const float* coef, const float* env,
                                     const int* tgt_ptr, const float* res, float* out,
                                     int64_t N, int64_t E, int64_t C, int64_t n_in,
                                     int env_first, float div, hipStream_t stream) {
  Lanes ln;
  TTA_CHECK_ARG(C > 0 && C % 4 == 0 && lanes_for(C, ln),
                "tta_rotate_env_segsum: unsupported channel count C=%lld", (long long)C);
  TTA_CHECK_ARG(n_in == 9 || n_in == 3, "tta_rotate_env_segsum: n_in must be 9 or 3");
  TTA_CHECK_ARG(N >= 0 && E >= 0 && N < (1ll << 31) && E < (1ll << 31),
                "tta_rotate_env_segsum: bad sizes");
  TTA_CHECK_ARG(div != 0.f, "tta_rotate_env_segsum: zero divisor");
  if (N == 0) return tta::kOk;
  TTA_CHECK_ARG(coef && env && tgt_ptr && out && (m || E == 0), "tta_rotate_env_segsum: null pointer");
  const unsigned blocks = tta_blocks(N * ln.G, 256);
#define TTA_LAUNCH_SEG(NIN, EF)                                                                \
  hipLaunchKernelGGL((k_rotate_env_segsum<NIN, EF>), dim3(blocks), dim3(256), 0, stream, m, coef, \
                     env, tgt_ptr, res, out, (int)N, (int)C, div, ln)
  if (n_in == 9 && env_first) TTA_LAUNCH_SEG(9, true);
  else if (n_in == 9) TTA_LAUNCH_SEG(9, false);
  else if (env_first) TTA_LAUNCH_SEG(3, true);
  else TTA_LAUNCH_SEG(3, false);
#undef TTA_LAUNCH_SEG
  TTA_CHECK_LAUNCH("tta_rotate_env_segsum");
  return tta::kOk;
}

extern "C" int tta_rotate_env_segsum_bw(const float* g_node, const int* tgt, const float* m,
                                        const float* coef, const float* env, float* g_m,
                                        float* g_coef, float* g_env, int64_t N, int64_t E,
                                        int64_t C, int64_t n_in, int env_first, float div,
                                        hipStream_t stream) {
  Lanes ln;
  TTA_CHECK_ARG(C > 0 && C % 4 == 0 && lanes_for(C, ln),
                "tta_rotate_env_segsum_bw: unsupported channel count C=%lld", (long long)C);
  TTA_CHECK_ARG(n_in == 9 || n_in == 3, "tta_rotate_env_segsum_bw: n_in must be 9 or 3");
  TTA_CHECK_ARG(E >= 0 && N >= 0 && E < (1ll << 31), "tta_rotate_env_segsum_bw: bad sizes");
  TTA_CHECK_ARG(div != 0.f, "tta_rotate_env_segsum_bw: zero divisor");
  if (E == 0) return tta::kOk;
  TTA_CHECK_ARG(g_node && tgt && m && coef && env && g_m && g_coef && g_env,
                "tta_rotate_env_segsum_bw: null pointer");
  const unsigned blocks = tta_blocks(E * ln.G, 256);
#define TTA_LAUNCH_SEGBW(NIN, EF)                                                               \
  hipLaunchKernelGGL((k_rotate_env_segsum_bw<NIN, EF>), dim3(blocks), dim3(256), 0, stream,     \
                     g_node, tgt, m, coef, env, g_m, g_coef, g_env, (int)E, (int)C, div, ln)
  if (n_in == 9 && env_first) TTA_LAUNCH_SEGBW(9, true);
  else if (n_in == 9) TTA_LAUNCH_SEGBW(9, false);
  else if (env_first) TTA_LAUNCH_SEGBW(3, true);
  else TTA_LAUNCH_SEGBW(3, false);
#undef TTA_LAUNCH_SEGBW
  TTA_CHECK_LAUNCH("tta_rotate_env_segsum_bw");
  return tta::kOk;
}

extern "C" int tta_node_gather_sum(const float* g_mcat, const int* src_ptr, const int* src_perm,
                                   const int* tgt_ptr, const float* res, float* out, int64_t N,
                                   int64_t E, int64_t C, hipStream_t stream) {
  Lanes ln;
  TTA_CHECK_ARG(C > 0 && C % 4 == 0 && lanes_for(C, ln),
                "tta_node_gather_sum: unsupported channel count C=%lld", (long long)C);
  TTA_CHECK_ARG(N >= 0 && E >= 0 && N < (1ll << 31), "tta_node_gather_sum: bad sizes");
  if (N == 0) return tta::kOk;
  TTA_CHECK_ARG(src_ptr && src_perm && tgt_ptr && out && (g_mcat || E == 0),
                "tta_node_gather_sum: null pointer");
  const unsigned blocks = tta_blocks(N * ln.G, 256);
  hipLaunchKernelGGL(k_node_gather_sum, dim3(blocks), dim3(256), 0, stream, g_mcat, src_ptr,
                     src_perm, tgt_ptr, res, out, (int)N, (int)C, ln);
  TTA_CHECK_LAUNCH("tta_node_gather_sum");
  return tta::kOk;
}
