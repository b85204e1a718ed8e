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
// Work mapping: one wavefront per edge (per node for the segmented sums).  The edge index is
// wave-uniform, so the 35 coefficients, the envelope and the src/tgt indices live in scalar
// registers.  The 64 lanes cover one coefficient row of W channels with V-wide vectors
// (V = 4, 2 or 1 so that W / V <= 64 where possible; wider rows loop).  Channel reductions
// (coefficient adjoints, envelope adjoint) are DPP butterflies inside each 16-lane row followed by
// a 4-entry LDS transpose; every output is written by exactly one lane with a plain store: no
// float atomics, deterministic results.
#include "common.h"

namespace {

constexpr int NSPH = 9;
constexpr int NNZ = 35;
constexpr int WAVES = 4;  // wavefronts per 256-thread block

template <int V>
struct VecT;
template <>
struct VecT<1> {
  typedef float T;
};
template <>
struct VecT<2> {
  typedef float T __attribute__((ext_vector_type(2)));
};
template <>
struct VecT<4> {
  typedef float T __attribute__((ext_vector_type(4)));
};

template <int V>
__device__ __forceinline__ typename VecT<V>::T ldv(const float* p) {
  return *reinterpret_cast<const typename VecT<V>::T*>(p);
}
// Nontemporal load for rows read exactly once (the radial rows and the edge adjoint of the
// gather kernels), so they do not displace the gathered node rows in L2 (-3 % on both kernels).
template <int V>
__device__ __forceinline__ typename VecT<V>::T ldv_nt(const float* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const typename VecT<V>::T*>(p));
}
// Streaming (nontemporal) stores: every edge-level output here is far larger than the L2 and is
// consumed by a later kernel, so allocating it in the cache only evicts the gathered node rows
// (measured on the C3 step: k_node_gather_sum -20 %, k_rotate_env_segsum -14 %,
// k_gather_rotate_bw -4 %).
template <int V>
__device__ __forceinline__ void stv(float* p, typename VecT<V>::T v) {
  __builtin_nontemporal_store(v, reinterpret_cast<typename VecT<V>::T*>(p));
}
template <int V>
__device__ __forceinline__ typename VecT<V>::T zv() {
  return typename VecT<V>::T(0.f);
}
template <int V>
__device__ __forceinline__ float hsum(typename VecT<V>::T v) {
  if constexpr (V == 1) {
    return v;
  } else if constexpr (V == 2) {
    return v[0] + v[1];
  } else {
    return (v[0] + v[1]) + (v[2] + v[3]);
  }
}

// out[m] = sum_j W[m, j] in[j]   (node SH -> edge frame; also the adjoint of the inverse rotation)
template <class T>
__device__ __forceinline__ void rot_fwd(const float* c, const T* in, T* out) {
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
template <int NIN, class T>
__device__ __forceinline__ void rot_inv(const float* c, const T* in, T* out) {
  out[0] = c[0] * in[0];
#pragma unroll
  for (int q = 0; q < 3; ++q) {
    T v = c[1 + q] * in[1];
    if (NIN > 3) v = v + c[9 + q] * in[3] + c[17 + q] * in[5];
    out[1 + q] = v;
  }
#pragma unroll
  for (int q = 0; q < 5; ++q) {
    T v = c[4 + q] * in[2];
    if (NIN > 3) v = v + c[12 + q] * in[4] + c[20 + q] * in[6] + c[25 + q] * in[7] + c[30 + q] * in[8];
    out[4 + q] = v;
  }
}

// Coefficient adjoint partials: gc[k] += <a[m_k], b[j_k]> over this lane's channels, where a is
// the m-primed-side tensor and b the natural-side tensor.  Only k with m_k < NIN.
template <int NIN, int V>
__device__ __forceinline__ void coef_partials(const typename VecT<V>::T* a,
                                              const typename VecT<V>::T* b, float* gc) {
  gc[0] += hsum<V>(a[0] * b[0]);
  const int m1[3] = {1, 3, 5}, k1[3] = {1, 9, 17};
#pragma unroll
  for (int r = 0; r < 3; ++r) {
    if (m1[r] >= NIN) continue;
#pragma unroll
    for (int q = 0; q < 3; ++q) gc[k1[r] + q] += hsum<V>(a[m1[r]] * b[1 + q]);
  }
  const int m2[5] = {2, 4, 6, 7, 8}, k2[5] = {4, 12, 20, 25, 30};
#pragma unroll
  for (int r = 0; r < 5; ++r) {
    if (m2[r] >= NIN) continue;
#pragma unroll
    for (int q = 0; q < 5; ++q) gc[k2[r] + q] += hsum<V>(a[m2[r]] * b[4 + q]);
  }
}

// Radial block of each m-primed coefficient: m0 {0,1,2} own blocks 0..2; the m=+-1 real/imag
// pairs (3,5) and (4,6) share blocks 3 and 4; the m=+-2 pair (7,8) shares block 5
// (so2.py:197-209: the radial output is duplicated as [m0 | m1 | m1 | m2 | m2]).
__device__ __forceinline__ int rad_block(int m) {
  const int rb[9] = {0, 1, 2, 3, 4, 3, 4, 5, 5};
  return rb[m];
}

template <int CTRL>
__device__ __forceinline__ float dpp_add(float v) {
  return v + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, true));
}

// Sums v[i] over the 64 lanes of the wave; afterwards lane i (< NV) holds total i.  DPP
// butterflies (quad xor 1, quad xor 2, half-row mirror, row mirror) leave each 16-lane row's sum in
// every lane of the row; the four row sums meet in a per-wave LDS slot `lds` [NV][4].
template <int NV>
__device__ __forceinline__ float wave_sums(float* v, float* lds, int lane) {
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    float x = v[i];
    x = dpp_add<0xB1>(x);   // quad_perm [1,0,3,2]
    x = dpp_add<0x4E>(x);   // quad_perm [2,3,0,1]
    x = dpp_add<0x141>(x);  // row_half_mirror
    x = dpp_add<0x140>(x);  // row_mirror
    v[i] = x;
  }
  if ((lane & 15) == 0) {
#pragma unroll
    for (int i = 0; i < NV; ++i) lds[i * 4 + (lane >> 4)] = v[i];
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  float t = 0.f;
  if (lane < NV) t = (lds[lane * 4] + lds[lane * 4 + 1]) + (lds[lane * 4 + 2] + lds[lane * 4 + 3]);
  return t;
}

// The same sums as a reduce-scatter by recursive halving: six exchange steps, each pairing a lane
// with a partner (lane xor 32, 16, 15, 7, 3, 1: v_permlane32_swap, v_permlane16_swap, DPP
// row_mirror, row_half_mirror and two quad permutations) and halving the values a lane carries
// (the lane keeps the lower or upper half of its slots by one lane bit: 5, 4, 3, 2, 1, 0 -- the
// bits the later partners leave alone), so after the six steps a value's 64 lane partials are
// summed in one lane: about 2.5 instructions per value against 5 and an LDS round trip.
// halving_index(lane) is the value a lane ends with, or -1 (lanes past the NV values hold 0).
template <int NV>
struct Halving {
  static_assert(NV >= 1 && NV <= 64, "1..64 values");
  static constexpr int n0 = NV, h1 = (n0 + 1) / 2, h2 = (h1 + 1) / 2, h3 = (h2 + 1) / 2,
                       h4 = (h3 + 1) / 2, h5 = (h4 + 1) / 2, h6 = (h5 + 1) / 2;
};

template <int NV>
__device__ __forceinline__ int halving_index(int lane) {
  typedef Halving<NV> H;
  const int size[6] = {H::n0, H::h1, H::h2, H::h3, H::h4, H::h5};  // each step's input slots
  const int half[6] = {H::h1, H::h2, H::h3, H::h4, H::h5, H::h6};
  const int bit[6] = {5, 4, 3, 2, 1, 0};
  int j = 0;  // the slot kept after the last step, traced back to the step's input
  for (int st = 5; st >= 0; --st) {
    j += ((lane >> bit[st]) & 1) * half[st];
    if (j >= size[st]) return -1;
  }
  return j;
}

// one step over lanes paired by a swap builtin: r[0] + r[1] is the pair's sum of the kept slot
template <int N, int HALF, bool X16>
__device__ __forceinline__ void halve_swap(const float* in, float* out) {
#pragma unroll
  for (int j = 0; j < HALF; ++j) {
    const unsigned a = __float_as_uint(in[j]), b = j + HALF < N ? __float_as_uint(in[j + HALF]) : 0u;
    const auto r = X16 ? __builtin_amdgcn_permlane16_swap(a, b, false, false)
                       : __builtin_amdgcn_permlane32_swap(a, b, false, false);
    out[j] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  }
}

// one step over lanes paired by a DPP permutation CTRL; `upper`: this lane keeps the upper half
template <int N, int HALF, int CTRL>
__device__ __forceinline__ void halve_dpp(const float* in, float* out, bool upper) {
#pragma unroll
  for (int j = 0; j < HALF; ++j) {
    const float a = in[j], b = j + HALF < N ? in[j + HALF] : 0.f;
    const float keep = upper ? b : a, send = upper ? a : b;
    out[j] = keep + __int_as_float(
                        __builtin_amdgcn_update_dpp(0, __float_as_int(send), CTRL, 0xF, 0xF, true));
  }
}

template <int NV>
__device__ __forceinline__ float halving_sums(const float* v, int lane) {
  typedef Halving<NV> H;
  float a[H::h1], b[H::h2], c[H::h3], d[H::h4], e[H::h5], f[H::h6];
  halve_swap<H::n0, H::h1, false>(v, a);                // lane ^ 32, keeps by bit 5
  halve_swap<H::h1, H::h2, true>(a, b);                 // lane ^ 16, bit 4
  halve_dpp<H::h2, H::h3, 0x140>(b, c, lane & 8);       // row_mirror: lane ^ 15, bit 3
  halve_dpp<H::h3, H::h4, 0x141>(c, d, lane & 4);       // row_half_mirror: lane ^ 7, bit 2
  halve_dpp<H::h4, H::h5, 0x1B>(d, e, lane & 2);        // quad_perm [3,2,1,0]: lane ^ 3, bit 1
  halve_dpp<H::h5, H::h6, 0xB1>(e, f, lane & 1);        // quad_perm [1,0,3,2]: lane ^ 1, bit 0
  return f[0];
}

__device__ __forceinline__ int wave_uniform(int v) { return __builtin_amdgcn_readfirstlane(v); }

__device__ __forceinline__ void load_coef(const float* __restrict__ coef, int64_t e, float* c) {
  const float* p = coef + e * NNZ;
#pragma unroll
  for (int k = 0; k < NNZ; ++k) c[k] = p[k];
}

// -------------------------------------------------------------------------------------------
// Forward: out[e, m, :] = (sum_j W[e,m,j] [x[src_e, j, :] | x[tgt_e, j, :]]) * rad[e, rb(m), :]
// (edgewise.py:52-69 gather + interleave + rotate, so2.py:263-277 radial multiply).
// HALVES = 1 gathers x[src_e] alone (row width C): a plain rotation of gathered source features.
template <int V, bool RAD, int HALVES = 2>
__global__ __launch_bounds__(256) void k_gather_rotate(const float* __restrict__ x,
                                                       const int* __restrict__ src,
                                                       const int* __restrict__ tgt,
                                                       const float* __restrict__ coef,
                                                       const float* __restrict__ rad,
                                                       float* __restrict__ out, int E, int C) {
  typedef typename VecT<V>::T T;
  const int lane = threadIdx.x & 63;
  const int e = wave_uniform(blockIdx.x * WAVES + (threadIdx.x >> 6));
  if (e >= E) return;
  const int W = HALVES * C, nq = W / V, cq = C / V;
  float c[NNZ];
  load_coef(coef, e, c);
  const int64_t s = wave_uniform(src[e]), t = HALVES == 2 ? wave_uniform(tgt[e]) : 0;
  for (int q = lane; q < nq; q += 64) {
    const float* row = (HALVES == 1 || q < cq) ? x + s * NSPH * C + V * q
                                               : x + t * NSPH * C + V * (q - cq);
    T in[NSPH], o[NSPH];
#pragma unroll
    for (int j = 0; j < NSPH; ++j) in[j] = ldv<V>(row + j * C);
    rot_fwd(c, in, o);
    float* orow = out + (int64_t)e * NSPH * W + V * q;
#pragma unroll
    for (int m = 0; m < NSPH; ++m) {
      T v = o[m];
      if (RAD) v = v * ldv_nt<V>(rad + (int64_t)e * 6 * W + rad_block(m) * W + V * q);
      stv<V>(orow + m * W, v);
    }
  }
}

// -------------------------------------------------------------------------------------------
// Backward of k_gather_rotate.  Recomputes the gathered input and the rotation instead of
// storing them.  Writes g_mcat [E, 9, 2C] (adjoint of the interleaved gather, scattered to
// nodes by k_node_gather_sum), g_rad [E, 6, 2C] (adjoint at the radial output, duplicate blocks
// collapsed) and accumulates the coefficient adjoint g_coef[e, k] += <g_mrot[m_k], m_cat[j_k]>
// (rotation.py:225-260 semantics).  HALVES = 1: source-only gather of row width C; g_mcat may then
// be NULL (only the coefficient adjoint is wanted).
template <int V, bool RAD, int HALVES = 2>
__global__ __launch_bounds__(256) void k_gather_rotate_bw(
    const float* __restrict__ g_xf, const float* __restrict__ rad, const float* __restrict__ x,
    const int* __restrict__ src, const int* __restrict__ tgt, const float* __restrict__ coef,
    float* __restrict__ g_rad, float* __restrict__ g_mcat, float* __restrict__ g_coef, int E,
    int C) {
  typedef typename VecT<V>::T T;
  __shared__ float red[WAVES][NNZ * 4];
  const int lane = threadIdx.x & 63;
  const int w = threadIdx.x >> 6;
  const int e = wave_uniform(blockIdx.x * WAVES + w);
  if (e >= E) return;
  const int W = HALVES * C, nq = W / V, cq = C / V;
  float c[NNZ];
  load_coef(coef, e, c);
  float gc[NNZ];
#pragma unroll
  for (int k = 0; k < NNZ; ++k) gc[k] = 0.f;
  const int64_t s = wave_uniform(src[e]), t = HALVES == 2 ? wave_uniform(tgt[e]) : 0;
  const int64_t eo = (int64_t)e * NSPH * W;
  for (int q = lane; q < nq; q += 64) {
    const float* row = (HALVES == 1 || q < cq) ? x + s * NSPH * C + V * q
                                               : x + t * NSPH * C + V * (q - cq);
    T in[NSPH], gm[NSPH];
#pragma unroll
    for (int j = 0; j < NSPH; ++j) in[j] = ldv<V>(row + j * C);
#pragma unroll
    for (int m = 0; m < NSPH; ++m) gm[m] = ldv_nt<V>(g_xf + eo + m * W + V * q);
    if (RAD) {
      const float* rr = rad + (int64_t)e * 6 * W + V * q;
      float* gr = g_rad + (int64_t)e * 6 * W + V * q;
      T mr[NSPH];
      rot_fwd(c, in, mr);
      // g_rad[b] = sum over the coefficients sharing radial block b (collapse the duplicates)
      stv<V>(gr + 0 * W, gm[0] * mr[0]);
      stv<V>(gr + 1 * W, gm[1] * mr[1]);
      stv<V>(gr + 2 * W, gm[2] * mr[2]);
      stv<V>(gr + 3 * W, gm[3] * mr[3] + gm[5] * mr[5]);
      stv<V>(gr + 4 * W, gm[4] * mr[4] + gm[6] * mr[6]);
      stv<V>(gr + 5 * W, gm[7] * mr[7] + gm[8] * mr[8]);
#pragma unroll
      for (int m = 0; m < NSPH; ++m) gm[m] = gm[m] * ldv_nt<V>(rr + rad_block(m) * W);
    }
    if (g_mcat) {
      T gi[NSPH];
      rot_inv<9>(c, gm, gi);
#pragma unroll
      for (int j = 0; j < NSPH; ++j) stv<V>(g_mcat + eo + j * W + V * q, gi[j]);
    }
    coef_partials<9, V>(gm, in, gc);
  }
  const float tot = wave_sums<NNZ>(gc, red[w], lane);
  if (lane < NNZ) g_coef[(int64_t)e * NNZ + lane] += tot;
}

// k_gather_rotate_bw walked by destination: a 128-thread block per node n goes over its edges
// [tgt_ptr[n], tgt_ptr[n+1]) (edges sorted by destination); wave 0 takes the source half of the
// channels (x[src_e] rows), wave 1 the destination half (x[n] rows).  Per edge as
// k_gather_rotate_bw (RAD, two halves), except that the destination half of the adjoint g_mcat
// is not stored: wave 1 sums it over the node's edges in ascending order from zero -- the order
// of k_node_gather_sum's destination loop, so the sum is bit-identical -- and writes it to
// tsum[n] [9, C] (zeros for a node without edges).  The coefficient adjoint of an edge is each
// wave's channel sum, the two added in wave order (source half first).  Every channel of a half
// sits in one lane vector (C / V <= 64).
template <int V>
__global__ __launch_bounds__(128) void k_gather_rotate_bw_dst(
    const float* __restrict__ g_xf, const float* __restrict__ rad, const float* __restrict__ x,
    const int* __restrict__ src, const int* __restrict__ tgt_ptr, const float* __restrict__ coef,
    float* __restrict__ g_rad, float* __restrict__ g_mcat, float* __restrict__ g_coef,
    float* __restrict__ tsum, int N, int C) {
  typedef typename VecT<V>::T T;
  __shared__ float red[2][NNZ * 4];
  __shared__ float half1[NNZ];
  const int lane = threadIdx.x & 63;
  const int h = threadIdx.x >> 6;  // channel half: 0 source, 1 destination
  const int n = blockIdx.x;
  if (n >= N) return;
  const int W = 2 * C, cq = C / V, q = lane;
  const bool active = q < cq;
  const int e0 = tgt_ptr[n], e1 = tgt_ptr[n + 1];
  const int co = h * C + V * q;  // this lane's first channel within a 2C row
  T b[NSPH];
#pragma unroll
  for (int j = 0; j < NSPH; ++j) b[j] = zv<V>();
  for (int e = e0; e < e1; ++e) {
    float c[NNZ];
    load_coef(coef, e, c);
    float gc[NNZ];
#pragma unroll
    for (int k = 0; k < NNZ; ++k) gc[k] = 0.f;
    const float gco = (h == 0 && lane < NNZ) ? g_coef[(int64_t)e * NNZ + lane] : 0.f;
    if (active) {
      const int64_t s = wave_uniform(src[e]);
      const int64_t eo = (int64_t)e * NSPH * W;
      const float* row = h == 0 ? x + s * NSPH * C + V * q : x + (int64_t)n * NSPH * C + V * q;
      T in[NSPH], gm[NSPH], mr[NSPH];
#pragma unroll
      for (int j = 0; j < NSPH; ++j) in[j] = ldv<V>(row + j * C);
#pragma unroll
      for (int m = 0; m < NSPH; ++m) gm[m] = ldv_nt<V>(g_xf + eo + m * W + co);
      rot_fwd(c, in, mr);
      float* grp = g_rad + (int64_t)e * 6 * W + co;
      stv<V>(grp + 0 * W, gm[0] * mr[0]);
      stv<V>(grp + 1 * W, gm[1] * mr[1]);
      stv<V>(grp + 2 * W, gm[2] * mr[2]);
      stv<V>(grp + 3 * W, gm[3] * mr[3] + gm[5] * mr[5]);
      stv<V>(grp + 4 * W, gm[4] * mr[4] + gm[6] * mr[6]);
      stv<V>(grp + 5 * W, gm[7] * mr[7] + gm[8] * mr[8]);
      const float* rp = rad + (int64_t)e * 6 * W + co;
#pragma unroll
      for (int m = 0; m < NSPH; ++m) gm[m] = gm[m] * ldv_nt<V>(rp + rad_block(m) * W);
      T gi[NSPH];
      rot_inv<9>(c, gm, gi);
      if (h == 1) {
#pragma unroll
        for (int j = 0; j < NSPH; ++j) b[j] = b[j] + gi[j];
      } else {
#pragma unroll
        for (int j = 0; j < NSPH; ++j) stv<V>(g_mcat + eo + j * W + co, gi[j]);
      }
      coef_partials<9, V>(gm, in, gc);
    }
    const float tot = wave_sums<NNZ>(gc, red[h], lane);
    if (h == 1 && lane < NNZ) half1[lane] = tot;
    __syncthreads();
    if (h == 0 && lane < NNZ) g_coef[(int64_t)e * NNZ + lane] = gco + (tot + half1[lane]);
    __syncthreads();
  }
  if (h == 1 && active) {
#pragma unroll
    for (int j = 0; j < NSPH; ++j) stv<V>(tsum + (int64_t)n * NSPH * C + j * C + V * q, b[j]);
  }
}

// The same backward walked from both ends of every edge, so that the adjoint of the interleaved
// gather never goes to memory: k_gather_rotate_bw_walk<V, false> takes the source half of each
// edge's channels ([0, C)) from its source node (edges through the source CSR, src_perm order),
// <V, true> the destination half ([C, 2C)) from its destination node (the contiguous destination
// segment).  One wavefront per node: the node's own row x[n] is loaded once (not gathered per
// edge), and the node's half of the gather adjoint is summed in registers over its edges in walk
// order from zero -- the source walk's sum is the source loop of k_node_gather_sum, the
// destination walk's that of k_gather_rotate_bw_dst -- and the destination walk writes
// out[n] = (source sum + destination sum) (+ res), the order of k_node_gather_sum.  Per edge
// the arithmetic is that of k_gather_rotate_bw_dst's wave for the half, so g_rad and the node
// adjoint are bit-identical to it; the coefficient adjoint's channel sum of the source half goes
// to coef_half [E, 35] and the destination walk accumulates g_coef = g_coef + (source half +
// destination half), its grouping too (each half's channel sum runs across lanes by recursive
// halving, so g_coef matches k_gather_rotate_bw_dst's to fp32 rounding).
template <int V, bool TGT>
__global__ __launch_bounds__(256) void k_gather_rotate_bw_walk(
    const float* __restrict__ g_xf, const float* __restrict__ rad, const float* __restrict__ x,
    const int* __restrict__ ptr, const int* __restrict__ perm, const float* __restrict__ coef,
    float* __restrict__ g_rad, float* __restrict__ g_coef, float* __restrict__ coef_half,
    const float* __restrict__ ssum, const float* __restrict__ res, float* __restrict__ out,
    int N, int C) {
  typedef typename VecT<V>::T T;
  const int lane = threadIdx.x & 63;
  const int w = threadIdx.x >> 6;
  const int n = wave_uniform(blockIdx.x * WAVES + w);
  const int ki = halving_index<NNZ>(lane);  // the coefficient whose sum this lane ends with
  const int kl = ki < 0 ? 0 : ki;
  if (n >= N) return;
  const int W = 2 * C, cq = C / V, q = lane;
  const bool active = q < cq;
  const int qq = active ? q : 0;  // idle lanes (C < 64 V) load channel 0 and store nothing
  const int co = (TGT ? C : 0) + V * qq;  // this lane's first channel within a 2C row
  const int k0 = wave_uniform(ptr[n]), k1 = wave_uniform(ptr[n + 1]);
  T in[NSPH], acc[NSPH];
#pragma unroll
  for (int j = 0; j < NSPH; ++j) {
    in[j] = ldv<V>(x + (int64_t)n * NSPH * C + j * C + V * qq);
    acc[j] = zv<V>();
  }
  for (int k = k0; k < k1; ++k) {
    const int64_t e = TGT ? k : wave_uniform(perm[k]);
    float c[NNZ];
    load_coef(coef, e, c);
    float gc[NNZ];
#pragma unroll
    for (int kk = 0; kk < NNZ; ++kk) gc[kk] = 0.f;
    // destination walk: the coefficient adjoint so far and the source walk's channel sum
    const float before = TGT ? g_coef[e * NNZ + kl] : 0.f;
    const float half0 = TGT ? coef_half[e * NNZ + kl] : 0.f;
    if (active) {
      const int64_t eo = e * NSPH * W + co;
      T gm[NSPH], mr[NSPH];
#pragma unroll
      for (int m = 0; m < NSPH; ++m) gm[m] = ldv_nt<V>(g_xf + eo + m * W);
      rot_fwd(c, in, mr);
      float* grp = g_rad + e * 6 * W + co;
      stv<V>(grp + 0 * W, gm[0] * mr[0]);
      stv<V>(grp + 1 * W, gm[1] * mr[1]);
      stv<V>(grp + 2 * W, gm[2] * mr[2]);
      stv<V>(grp + 3 * W, gm[3] * mr[3] + gm[5] * mr[5]);
      stv<V>(grp + 4 * W, gm[4] * mr[4] + gm[6] * mr[6]);
      stv<V>(grp + 5 * W, gm[7] * mr[7] + gm[8] * mr[8]);
      const float* rp = rad + e * 6 * W + co;
#pragma unroll
      for (int m = 0; m < NSPH; ++m) gm[m] = gm[m] * ldv_nt<V>(rp + rad_block(m) * W);
      T gi[NSPH];
      rot_inv<9>(c, gm, gi);
      {
        // every row rounded before it is added, as k_node_gather_sum adds the stored rows and
        // k_gather_rotate_bw_dst adds them in a later block (gi[0] is a bare product, which the
        // add would otherwise absorb into an fma)
#pragma clang fp contract(off)
#pragma unroll
        for (int j = 0; j < NSPH; ++j) acc[j] = acc[j] + gi[j];
      }
      coef_partials<9, V>(gm, in, gc);
    }
    const float tot = halving_sums<NNZ>(gc, lane);
    if (ki >= 0) {
      if (TGT)
        g_coef[e * NNZ + ki] = before + (half0 + tot);
      else
        coef_half[e * NNZ + ki] = tot;
    }
  }
  if (!active) return;
  const int64_t no = (int64_t)n * NSPH * C + V * q;
#pragma unroll
  for (int j = 0; j < NSPH; ++j) {
    if (!TGT) {
      stv<V>(out + no + j * C, acc[j]);
    } else {
      T v = ldv<V>(ssum + no + j * C) + acc[j];
      if (res) v = v + ldv<V>(res + no + j * C);
      stv<V>(out + no + j * C, v);
    }
  }
}

// -------------------------------------------------------------------------------------------
// Inverse rotation + envelope + destination-sorted segmented sum (+ residual):
//   out[n, j, :] = res[n, j, :] + sum_{e in [ptr[n], ptr[n+1])} contrib_e[j, :]
// ENV_FIRST (edgewise.py:72-86):  contrib = W^T (m[e] * env[e])
// otherwise (geometry.py:269-276, edge-degree init): contrib = (W^T pad(m[e])) * (env[e] / div)
// Edges of a segment are summed in ascending order starting from zero, then the residual is
// added: the order index_add_ followed by "+ x_res" uses.  One wave per node walks its edges in
// order; the loads of edge e + PF are issued before edge e is accumulated, so PF edges' worth of
// loads are in flight: each edge's message rows, and its 35 coefficients and envelope in one
// coalesced load (lane k < 35 holds coefficient k, lane 35 the envelope) whose values reach the
// arithmetic through v_readlane with constant lane indices (scalar loads per edge would put a
// scalar-memory round trip on every edge of the chain).
// PF: 4 edges in flight, 2 for wide rows (V NIN > 18 floats per lane per edge) to stay within
// 256 registers.  Every slot refill issues the same loads unconditionally (the edge index clamped
// to the segment's last edge, the clamped edge's values then unused), so the compiler's wait
// counts stay exact: a conditional load would make it wait for all loads at the join.
constexpr int kSegPF = 4;

template <int V, int NIN, bool ENV_FIRST>
__global__ __launch_bounds__(256) void k_rotate_env_segsum(
    const float* __restrict__ m, const float* __restrict__ coef, const float* __restrict__ env,
    const int* __restrict__ ptr, const float* __restrict__ res, float* __restrict__ out, int N,
    int C, float div) {
  typedef typename VecT<V>::T T;
  const int lane = threadIdx.x & 63;
  const int n = wave_uniform(blockIdx.x * WAVES + (threadIdx.x >> 6));
  if (n >= N) return;
  const int e0 = wave_uniform(ptr[n]), e1 = wave_uniform(ptr[n + 1]);
  const int nq = C / V;
  const float rdiv = 1.f / div;
  constexpr int PF = V * NIN > 18 ? 2 : kSegPF;
  // lane k < 35 loads coefficient k of the edge, the other lanes its envelope (lane 35's copy is
  // the one read): one load instruction, no branch
  const int ce_off = lane < NNZ ? lane : 0;
  auto load_ce = [&](int e) -> float {
    const float* p = lane < NNZ ? coef + (int64_t)e * NNZ + ce_off : env + e;
    return *p;
  };
  for (int q0 = 0; q0 < nq; q0 += 64) {
    // every lane runs the loop, also past the channel rows (its row loads then read channel 0
    // and it stores nothing), so that lanes 0..35 all take part in the coefficient loads
    const int q = q0 + lane;
    const bool qv = q < nq;
    const int qq = qv ? q : 0;
    T acc[NSPH];
#pragma unroll
    for (int j = 0; j < NSPH; ++j) acc[j] = zv<V>();
    if (e0 < e1) {
      T rows[PF][NIN];
      float ce[PF];
      auto load_slot = [&](int s, int e) {
        e = min(e, e1 - 1);
        ce[s] = load_ce(e);
#pragma unroll
        for (int mm = 0; mm < NIN; ++mm) rows[s][mm] = ldv<V>(m + (int64_t)e * NIN * C + mm * C + V * qq);
      };
#pragma unroll
      for (int s = 0; s < PF; ++s) load_slot(s, e0 + s);
      for (int eb = e0; eb < e1; eb += PF) {
#pragma unroll
        for (int s = 0; s < PF; ++s) {
          const int e = eb + s;
          T in[NSPH];
#pragma unroll
          for (int mm = 0; mm < NSPH; ++mm) in[mm] = zv<V>();
#pragma unroll
          for (int mm = 0; mm < NIN; ++mm) in[mm] = rows[s][mm];
          float c[NNZ];
          const int cev = __float_as_int(ce[s]);
#pragma unroll
          for (int k = 0; k < NNZ; ++k) c[k] = __int_as_float(__builtin_amdgcn_readlane(cev, k));
          const float ev = __int_as_float(__builtin_amdgcn_readlane(cev, NNZ));
          // refill this slot with edge e + PF before the arithmetic of edge e
          load_slot(s, e + PF);
          if (e < e1) {  // wave-uniform
            if (ENV_FIRST) {
#pragma unroll
              for (int mm = 0; mm < NIN; ++mm) in[mm] = in[mm] * ev;
            }
            T o[NSPH];
            rot_inv<NIN>(c, in, o);
            // edge-degree scaling: one per-edge factor env / div (a division per element made
            // this variant VALU-bound; the factor rounds once, so values move by an ulp at most)
            const float sc = ENV_FIRST ? 1.f : ev * rdiv;
#pragma unroll
            for (int j = 0; j < NSPH; ++j) {
              T v = o[j];
              if (!ENV_FIRST) v = v * sc;
              acc[j] = acc[j] + v;
            }
          }
        }
      }
    }
    if (qv) {
#pragma unroll
      for (int j = 0; j < NSPH; ++j) {
        T v = acc[j];
        if (res) v = v + ldv<V>(res + (int64_t)n * NSPH * C + j * C + V * q);
        stv<V>(out + (int64_t)n * NSPH * C + j * C + V * q, v);
      }
    }
  }
}

// -------------------------------------------------------------------------------------------
// Backward of k_rotate_env_segsum for one edge (the scatter adjoint is a gather by tgt):
// ENV_FIRST (forces.py:366-376):
//   g_back = g_node[tgt]; g_env_in = W g_back; g_m = g_env_in * env;
//   g_env += <g_env_in, m>;  g_coef(m,j) += <g_back[j], m[m] * env>
// otherwise (edge-degree, forward v = (W^T pad(m)) * (env / div)):
//   g_v2 = g_node[tgt] (1 / div); g_v1 = g_v2 * env; g_env += <g_v2, W^T pad(m)>;
//   g_m = (W g_v1)[:NIN];  g_coef(m,j) += <g_v1[j], pad(m)[m]>
template <int V, int NIN, bool ENV_FIRST>
__global__ __launch_bounds__(256) void k_rotate_env_segsum_bw(
    const float* __restrict__ g_node, const int* __restrict__ tgt, const float* __restrict__ m,
    const float* __restrict__ coef, const float* __restrict__ env, float* __restrict__ g_m,
    float* __restrict__ g_coef, float* __restrict__ g_env, int E, int C, float div) {
  typedef typename VecT<V>::T T;
  const int lane = threadIdx.x & 63;
  const int w = threadIdx.x >> 6;
  const int e = wave_uniform(blockIdx.x * WAVES + w);
  if (e >= E) return;
  const int nq = C / V;
  float c[NNZ];
  load_coef(coef, e, c);
  const float ev = env[e];
  const int64_t t = wave_uniform(tgt[e]);
  const float rdiv = 1.f / div;
  float gc[NNZ + 1];  // 35 coefficient partials + the envelope partial
#pragma unroll
  for (int k = 0; k <= NNZ; ++k) gc[k] = 0.f;
  for (int q = lane; q < nq; q += 64) {
    T gb[NSPH], mi[NSPH];
#pragma unroll
    for (int j = 0; j < NSPH; ++j) gb[j] = ldv<V>(g_node + t * NSPH * C + j * C + V * q);
#pragma unroll
    for (int mm = 0; mm < NSPH; ++mm)
      mi[mm] = mm < NIN ? ldv<V>(m + (int64_t)e * NIN * C + mm * C + V * q) : zv<V>();
    if (ENV_FIRST) {
      T gin[NSPH], me[NSPH];
      rot_fwd(c, gb, gin);
#pragma unroll
      for (int mm = 0; mm < NSPH; ++mm) {
        me[mm] = mi[mm] * ev;
        if (mm >= NIN) continue;
        gc[NNZ] += hsum<V>(gin[mm] * mi[mm]);
        stv<V>(g_m + (int64_t)e * NIN * C + mm * C + V * q, gin[mm] * ev);
      }
      coef_partials<NIN, V>(me, gb, gc);
    } else {
      T v1[NSPH], g1[NSPH], gin[NSPH];
      rot_inv<NIN>(c, mi, v1);
#pragma unroll
      for (int j = 0; j < NSPH; ++j) {
        const T g2 = gb[j] * rdiv;  // (a division per element made this variant VALU-bound)
        gc[NNZ] += hsum<V>(g2 * v1[j]);
        g1[j] = g2 * ev;
      }
      rot_fwd(c, g1, gin);
#pragma unroll
      for (int mm = 0; mm < NIN; ++mm) stv<V>(g_m + (int64_t)e * NIN * C + mm * C + V * q, gin[mm]);
      coef_partials<NIN, V>(mi, g1, gc);
    }
  }
  // the 35 coefficient sums and the envelope's (value NNZ), each in one lane
  const float tot = halving_sums<NNZ + 1>(gc, lane);
  const int ki = halving_index<NNZ + 1>(lane);
  if (ki >= 0 && ki < NNZ) g_coef[(int64_t)e * NNZ + ki] += tot;
  if (ki == NNZ) g_env[e] += tot;
}

// -------------------------------------------------------------------------------------------
// Node adjoint of the interleaved src|tgt gather (forces.py:384-412):
//   g_x[n] = sum_{edges with src = n} g_mcat[e, :, 0:C] + sum_{edges with tgt = n} g_mcat[e, :, C:2C]
// src edges come through a src-sorted permutation (src_ptr / src_perm), tgt edges are the
// contiguous destination segments.  Optional residual: out = (src sum + tgt sum) + res.
template <int V>
__global__ __launch_bounds__(256) void k_node_gather_sum(
    const float* __restrict__ g_mcat, const int* __restrict__ src_ptr,
    const int* __restrict__ src_perm, const int* __restrict__ tgt_ptr,
    const float* __restrict__ res, float* __restrict__ out, int N, int C,
    const float* __restrict__ tsum = nullptr) {
  typedef typename VecT<V>::T T;
  const int lane = threadIdx.x & 63;
  const int n = wave_uniform(blockIdx.x * WAVES + (threadIdx.x >> 6));
  if (n >= N) return;
  const int W = 2 * C, nq = C / V;
  const int s0 = wave_uniform(src_ptr[n]), s1 = wave_uniform(src_ptr[n + 1]);
  const int t0 = tgt_ptr ? wave_uniform(tgt_ptr[n]) : 0;
  const int t1 = tgt_ptr ? wave_uniform(tgt_ptr[n + 1]) : 0;
  for (int q = lane; q < nq; q += 64) {
    T a[NSPH], b[NSPH];
#pragma unroll
    for (int j = 0; j < NSPH; ++j) a[j] = b[j] = zv<V>();
    for (int k = s0; k < s1; ++k) {
      const int64_t e = wave_uniform(src_perm[k]);
#pragma unroll
      for (int j = 0; j < NSPH; ++j) a[j] = a[j] + ldv<V>(g_mcat + e * NSPH * W + j * W + V * q);
    }
    if (tsum) {  // the destination sums, already formed by k_gather_rotate_bw_dst
#pragma unroll
      for (int j = 0; j < NSPH; ++j) b[j] = ldv<V>(tsum + (int64_t)n * NSPH * C + j * C + V * q);
    } else {
      for (int64_t e = t0; e < t1; ++e) {
#pragma unroll
        for (int j = 0; j < NSPH; ++j)
          b[j] = b[j] + ldv<V>(g_mcat + e * NSPH * W + j * W + C + V * q);
      }
    }
#pragma unroll
    for (int j = 0; j < NSPH; ++j) {
      T v = a[j] + b[j];
      if (res) v = v + ldv<V>(res + (int64_t)n * NSPH * C + j * C + V * q);
      stv<V>(out + (int64_t)n * NSPH * C + j * C + V * q, v);
    }
  }
}

// Vector width for a row of W channels (W a multiple of 4): the widest of 4, 2, 1 that still
// gives every one of the 64 lanes a vector (narrow rows leave lanes idle; wide rows loop).
int pick_v(int64_t W) {
  if (W >= 256) return 4;
  if (W >= 128) return 2;
  return 1;
}

unsigned wave_blocks(int64_t items) { return (unsigned)((items + WAVES - 1) / WAVES); }

}  // namespace

// =========================================================================== C ABI
#define TTA_V_DISPATCH(V, ...)       \
  do {                               \
    if (V == 4) {                    \
      constexpr int VV = 4;          \
      __VA_ARGS__;                   \
    } else if (V == 2) {             \
      constexpr int VV = 2;          \
      __VA_ARGS__;                   \
    } else {                         \
      constexpr int VV = 1;          \
      __VA_ARGS__;                   \
    }                                \
  } while (0)

extern "C" int tta_gather_rotate(const float* x, const int* src, const int* tgt,
                                 const float* coef, const float* rad, float* out, int64_t N,
                                 int64_t E, int64_t C, hipStream_t stream) {
  TTA_CHECK_ARG(C > 0 && C % 4 == 0 && C <= 4096,
                "tta_gather_rotate: unsupported channel count C=%lld", (long long)C);
  TTA_CHECK_ARG(E >= 0 && N >= 0 && E < (1ll << 31), "tta_gather_rotate: bad sizes");
  if (E == 0) return tta::kOk;
  TTA_CHECK_ARG(x && src && tgt && coef && out, "tta_gather_rotate: null pointer");
  const int V = pick_v(2 * C);  // divides C: C is a multiple of 4
  TTA_V_DISPATCH(V, {
    if (rad)
      hipLaunchKernelGGL((k_gather_rotate<VV, true>), dim3(wave_blocks(E)), dim3(256), 0, stream,
                         x, src, tgt, coef, rad, out, (int)E, (int)C);
    else
      hipLaunchKernelGGL((k_gather_rotate<VV, false>), dim3(wave_blocks(E)), dim3(256), 0,
                         stream, x, src, tgt, coef, rad, out, (int)E, (int)C);
  });
  TTA_CHECK_LAUNCH("tta_gather_rotate");
  return tta::kOk;
}

extern "C" int tta_gather_rotate_bw(const float* g_xf, const float* rad, const float* x,
                                    const int* src, const int* tgt, const float* coef,
                                    float* g_rad, float* g_mcat, float* g_coef, int64_t N,
                                    int64_t E, int64_t C, hipStream_t stream) {
  TTA_CHECK_ARG(C > 0 && C % 4 == 0 && C <= 4096,
                "tta_gather_rotate_bw: unsupported channel count C=%lld", (long long)C);
  TTA_CHECK_ARG(E >= 0 && N >= 0 && E < (1ll << 31), "tta_gather_rotate_bw: bad sizes");
  if (E == 0) return tta::kOk;
  TTA_CHECK_ARG(g_xf && x && src && tgt && coef && g_mcat && g_coef,
                "tta_gather_rotate_bw: null pointer");
  TTA_CHECK_ARG(!rad == !g_rad, "tta_gather_rotate_bw: rad and g_rad must be given together");
  const int V = pick_v(2 * C);
  TTA_V_DISPATCH(V, {
    if (rad)
      hipLaunchKernelGGL((k_gather_rotate_bw<VV, true>), dim3(wave_blocks(E)), dim3(256), 0,
                         stream, g_xf, rad, x, src, tgt, coef, g_rad, g_mcat, g_coef, (int)E,
                         (int)C);
    else
      hipLaunchKernelGGL((k_gather_rotate_bw<VV, false>), dim3(wave_blocks(E)), dim3(256), 0,
                         stream, g_xf, rad, x, src, tgt, coef, g_rad, g_mcat, g_coef, (int)E,
                         (int)C);
  });
  TTA_CHECK_LAUNCH("tta_gather_rotate_bw");
  return tta::kOk;
}

extern "C" int tta_gather_rotate_bw_dst(const float* g_xf, const float* rad, const float* x,
                                        const int* src, const int* tgt_ptr, const float* coef,
                                        float* g_rad, float* g_mcat, float* g_coef, float* tsum,
                                        int64_t N, int64_t E, int64_t C, hipStream_t stream) {
  TTA_CHECK_ARG(C > 0 && C % 4 == 0 && C / pick_v(C) <= 64,
                "tta_gather_rotate_bw_dst: channel count C=%lld needs C / V <= 64 "
                "(C <= 64, 128 or 256)",
                (long long)C);
  TTA_CHECK_ARG(E >= 0 && N >= 0 && E < (1ll << 31) && N < (1ll << 31),
                "tta_gather_rotate_bw_dst: bad sizes");
  if (N == 0) return tta::kOk;
  TTA_CHECK_ARG(tgt_ptr && tsum && (E == 0 || (g_xf && rad && x && src && coef && g_rad &&
                                                g_mcat && g_coef)),
                "tta_gather_rotate_bw_dst: null pointer");
  const int V = pick_v(C);
  TTA_V_DISPATCH(V, {
    hipLaunchKernelGGL((k_gather_rotate_bw_dst<VV>), dim3((unsigned)N), dim3(128), 0, stream,
                       g_xf, rad, x, src, tgt_ptr, coef, g_rad, g_mcat, g_coef, tsum, (int)N,
                       (int)C);
  });
  TTA_CHECK_LAUNCH("tta_gather_rotate_bw_dst");
  return tta::kOk;
}

// The two walks of the rotation backward (k_gather_rotate_bw_walk); the source walk runs first.
static int bw_walk_check(int64_t N, int64_t E, int64_t C, const char* who) {
  TTA_CHECK_ARG(C > 0 && C % 4 == 0 && C / pick_v(C) <= 64,
                "%s: channel count C=%lld needs C / V <= 64 (C <= 64, 128 or 256)", who,
                (long long)C);
  TTA_CHECK_ARG(E >= 0 && N >= 0 && E < (1ll << 31) && N < (1ll << 31), "%s: bad sizes", who);
  return tta::kOk;
}

extern "C" int tta_gather_rotate_bw_srcwalk(const float* g_xf, const float* rad, const float* x,
                                            const int* src_ptr, const int* src_perm,
                                            const float* coef, float* g_rad, float* coef_half,
                                            float* ssum, int64_t N, int64_t E, int64_t C,
                                            hipStream_t stream) {
  const int rc = bw_walk_check(N, E, C, "tta_gather_rotate_bw_srcwalk");
  if (rc != tta::kOk || N == 0) return rc;
  TTA_CHECK_ARG(src_ptr && x && ssum && (E == 0 || (src_perm && g_xf && rad && coef && g_rad &&
                                                     coef_half)),
                "tta_gather_rotate_bw_srcwalk: null pointer");
  const int V = pick_v(C);
  TTA_V_DISPATCH(V, {
    hipLaunchKernelGGL((k_gather_rotate_bw_walk<VV, false>), dim3(wave_blocks(N)), dim3(256), 0,
                       stream, g_xf, rad, x, src_ptr, src_perm, coef, g_rad, nullptr, coef_half,
                       nullptr, nullptr, ssum, (int)N, (int)C);
  });
  TTA_CHECK_LAUNCH("tta_gather_rotate_bw_srcwalk");
  return tta::kOk;
}

extern "C" int tta_gather_rotate_bw_tgtwalk(const float* g_xf, const float* rad, const float* x,
                                            const int* tgt_ptr, const float* coef, float* g_rad,
                                            float* g_coef, const float* coef_half,
                                            const float* ssum, const float* res, float* out,
                                            int64_t N, int64_t E, int64_t C,
                                            hipStream_t stream) {
  const int rc = bw_walk_check(N, E, C, "tta_gather_rotate_bw_tgtwalk");
  if (rc != tta::kOk || N == 0) return rc;
  TTA_CHECK_ARG(tgt_ptr && x && ssum && out && (E == 0 || (g_xf && rad && coef && g_rad &&
                                                           g_coef && coef_half)),
                "tta_gather_rotate_bw_tgtwalk: null pointer");
  const int V = pick_v(C);
  TTA_V_DISPATCH(V, {
    hipLaunchKernelGGL((k_gather_rotate_bw_walk<VV, true>), dim3(wave_blocks(N)), dim3(256), 0,
                       stream, g_xf, rad, x, tgt_ptr, nullptr, coef, g_rad, g_coef,
                       const_cast<float*>(coef_half), ssum, res, out, (int)N, (int)C);
  });
  TTA_CHECK_LAUNCH("tta_gather_rotate_bw_tgtwalk");
  return tta::kOk;
}

extern "C" int tta_gather_rotate_src(const float* x, const int* src, const float* coef,
                                     float* out, int64_t N, int64_t E, int64_t C,
                                     hipStream_t stream) {
  TTA_CHECK_ARG(C > 0 && C % 4 == 0 && C <= 4096,
                "tta_gather_rotate_src: unsupported channel count C=%lld", (long long)C);
  TTA_CHECK_ARG(E >= 0 && N >= 0 && E < (1ll << 31), "tta_gather_rotate_src: bad sizes");
  if (E == 0) return tta::kOk;
  TTA_CHECK_ARG(x && src && coef && out, "tta_gather_rotate_src: null pointer");
  const int V = pick_v(C);
  TTA_V_DISPATCH(V, {
    hipLaunchKernelGGL((k_gather_rotate<VV, false, 1>), dim3(wave_blocks(E)), dim3(256), 0,
                       stream, x, src, nullptr, coef, nullptr, out, (int)E, (int)C);
  });
  TTA_CHECK_LAUNCH("tta_gather_rotate_src");
  return tta::kOk;
}

extern "C" int tta_gather_rotate_src_bw(const float* g_out, const float* x, const int* src,
                                        const float* coef, float* g_in, float* g_coef,
                                        int64_t N, int64_t E, int64_t C, hipStream_t stream) {
  TTA_CHECK_ARG(C > 0 && C % 4 == 0 && C <= 4096,
                "tta_gather_rotate_src_bw: unsupported channel count C=%lld", (long long)C);
  TTA_CHECK_ARG(E >= 0 && N >= 0 && E < (1ll << 31), "tta_gather_rotate_src_bw: bad sizes");
  if (E == 0) return tta::kOk;
  TTA_CHECK_ARG(g_out && x && src && coef && g_coef, "tta_gather_rotate_src_bw: null pointer");
  const int V = pick_v(C);
  TTA_V_DISPATCH(V, {
    hipLaunchKernelGGL((k_gather_rotate_bw<VV, false, 1>), dim3(wave_blocks(E)), dim3(256), 0,
                       stream, g_out, nullptr, x, src, nullptr, coef, nullptr, g_in, g_coef,
                       (int)E, (int)C);
  });
  TTA_CHECK_LAUNCH("tta_gather_rotate_src_bw");
  return tta::kOk;
}

extern "C" int tta_rotate_env_segsum(const float* m, const float* coef, const float* env,
                                     const int* tgt_ptr, const float* res, float* out,
                                     int64_t N, int64_t E, int64_t C, int64_t n_in,
                                     int env_first, float div, hipStream_t stream) {
  TTA_CHECK_ARG(C > 0 && C % 4 == 0 && C <= 4096,
                "tta_rotate_env_segsum: unsupported channel count C=%lld", (long long)C);
  TTA_CHECK_ARG(n_in == 9 || n_in == 3, "tta_rotate_env_segsum: n_in must be 9 or 3");
  TTA_CHECK_ARG(N >= 0 && E >= 0 && N < (1ll << 31) && E < (1ll << 31),
                "tta_rotate_env_segsum: bad sizes");
  TTA_CHECK_ARG(div != 0.f, "tta_rotate_env_segsum: zero divisor");
  if (N == 0) return tta::kOk;
  TTA_CHECK_ARG(coef && env && tgt_ptr && out && (m || E == 0), "tta_rotate_env_segsum: null pointer");
  const int V = pick_v(C);
  TTA_V_DISPATCH(V, {
    if (n_in == 9 && env_first)
      hipLaunchKernelGGL((k_rotate_env_segsum<VV, 9, true>), dim3(wave_blocks(N)), dim3(256), 0,
                         stream, m, coef, env, tgt_ptr, res, out, (int)N, (int)C, div);
    else if (n_in == 9)
      hipLaunchKernelGGL((k_rotate_env_segsum<VV, 9, false>), dim3(wave_blocks(N)), dim3(256), 0,
                         stream, m, coef, env, tgt_ptr, res, out, (int)N, (int)C, div);
    else if (env_first)
      hipLaunchKernelGGL((k_rotate_env_segsum<VV, 3, true>), dim3(wave_blocks(N)), dim3(256), 0,
                         stream, m, coef, env, tgt_ptr, res, out, (int)N, (int)C, div);
    else
      hipLaunchKernelGGL((k_rotate_env_segsum<VV, 3, false>), dim3(wave_blocks(N)), dim3(256), 0,
                         stream, m, coef, env, tgt_ptr, res, out, (int)N, (int)C, div);
  });
  TTA_CHECK_LAUNCH("tta_rotate_env_segsum");
  return tta::kOk;
}

extern "C" int tta_rotate_env_segsum_bw(const float* g_node, const int* tgt, const float* m,
                                        const float* coef, const float* env, float* g_m,
                                        float* g_coef, float* g_env, int64_t N, int64_t E,
                                        int64_t C, int64_t n_in, int env_first, float div,
                                        hipStream_t stream) {
  TTA_CHECK_ARG(C > 0 && C % 4 == 0 && C <= 4096,
                "tta_rotate_env_segsum_bw: unsupported channel count C=%lld", (long long)C);
  TTA_CHECK_ARG(n_in == 9 || n_in == 3, "tta_rotate_env_segsum_bw: n_in must be 9 or 3");
  TTA_CHECK_ARG(E >= 0 && N >= 0 && E < (1ll << 31), "tta_rotate_env_segsum_bw: bad sizes");
  TTA_CHECK_ARG(div != 0.f, "tta_rotate_env_segsum_bw: zero divisor");
  if (E == 0) return tta::kOk;
  TTA_CHECK_ARG(g_node && tgt && m && coef && env && g_m && g_coef && g_env,
                "tta_rotate_env_segsum_bw: null pointer");
  const int V = pick_v(C);
  TTA_V_DISPATCH(V, {
    if (n_in == 9 && env_first)
      hipLaunchKernelGGL((k_rotate_env_segsum_bw<VV, 9, true>), dim3(wave_blocks(E)), dim3(256),
                         0, stream, g_node, tgt, m, coef, env, g_m, g_coef, g_env, (int)E, (int)C,
                         div);
    else if (n_in == 9)
      hipLaunchKernelGGL((k_rotate_env_segsum_bw<VV, 9, false>), dim3(wave_blocks(E)), dim3(256),
                         0, stream, g_node, tgt, m, coef, env, g_m, g_coef, g_env, (int)E, (int)C,
                         div);
    else if (env_first)
      hipLaunchKernelGGL((k_rotate_env_segsum_bw<VV, 3, true>), dim3(wave_blocks(E)), dim3(256),
                         0, stream, g_node, tgt, m, coef, env, g_m, g_coef, g_env, (int)E, (int)C,
                         div);
    else
      hipLaunchKernelGGL((k_rotate_env_segsum_bw<VV, 3, false>), dim3(wave_blocks(E)), dim3(256),
                         0, stream, g_node, tgt, m, coef, env, g_m, g_coef, g_env, (int)E, (int)C,
                         div);
  });
  TTA_CHECK_LAUNCH("tta_rotate_env_segsum_bw");
  return tta::kOk;
}

extern "C" int tta_node_gather_sum_dst(const float* g_mcat, const int* src_ptr,
                                       const int* src_perm, const float* tsum, const float* res,
                                       float* out, int64_t N, int64_t E, int64_t C,
                                       hipStream_t stream) {
  TTA_CHECK_ARG(C > 0 && C % 4 == 0 && C <= 4096,
                "tta_node_gather_sum_dst: unsupported channel count C=%lld", (long long)C);
  TTA_CHECK_ARG(N >= 0 && E >= 0 && N < (1ll << 31), "tta_node_gather_sum_dst: bad sizes");
  if (N == 0) return tta::kOk;
  TTA_CHECK_ARG(src_ptr && src_perm && tsum && out && (g_mcat || E == 0),
                "tta_node_gather_sum_dst: null pointer");
  const int V = pick_v(C);
  TTA_V_DISPATCH(V, {
    hipLaunchKernelGGL((k_node_gather_sum<VV>), dim3(wave_blocks(N)), dim3(256), 0, stream,
                       g_mcat, src_ptr, src_perm, nullptr, res, out, (int)N, (int)C, tsum);
  });
  TTA_CHECK_LAUNCH("tta_node_gather_sum_dst");
  return tta::kOk;
}

extern "C" int tta_node_gather_sum(const float* g_mcat, const int* src_ptr, const int* src_perm,
                                   const int* tgt_ptr, const float* res, float* out, int64_t N,
                                   int64_t E, int64_t C, hipStream_t stream) {
  TTA_CHECK_ARG(C > 0 && C % 4 == 0 && C <= 4096,
                "tta_node_gather_sum: unsupported channel count C=%lld", (long long)C);
  TTA_CHECK_ARG(N >= 0 && E >= 0 && N < (1ll << 31), "tta_node_gather_sum: bad sizes");
  if (N == 0) return tta::kOk;
  TTA_CHECK_ARG(src_ptr && src_perm && tgt_ptr && out && (g_mcat || E == 0),
                "tta_node_gather_sum: null pointer");
  const int V = pick_v(C);
  TTA_V_DISPATCH(V, {
    hipLaunchKernelGGL((k_node_gather_sum<VV>), dim3(wave_blocks(N)), dim3(256), 0, stream,
                       g_mcat, src_ptr, src_perm, tgt_ptr, res, out, (int)N, (int)C);
  });
  TTA_CHECK_LAUNCH("tta_node_gather_sum");
  return tta::kOk;
}
