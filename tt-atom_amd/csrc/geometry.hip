// Edge geometry kernels: positions -> (edge vectors, distances, packed Wigner coefficients,
// radial features, envelope) and the reverse: coefficient / radial / envelope adjoints -> edge
// vector adjoints -> forces (deterministic CSR sums) and the symmetric virial.
//
// Reference: tt_atom/geometry.py:226-280 (forward terms) and the host autograd finish of
// forces.py:545-589 (here in closed form, geometry_math.h).
#include <mutex>

#include "common.h"
#include "geometry_math.h"

namespace {

// One thread per edge: ev = pos[src] - pos[tgt] (+ shift), dist = |ev|, coef = packed W(ev).
// The block's 256 coefficient rows (35 floats each) and edge vectors are staged in LDS and then
// stored with consecutive lanes on consecutive floats: a thread storing its own row would make
// each store instruction touch 64 cache lines.
__global__ __launch_bounds__(256) void k_edge_wigner(const float* __restrict__ pos,
                                                     const int* __restrict__ src,
                                                     const int* __restrict__ tgt,
                                                     const float* __restrict__ shift,
                                                     const float* __restrict__ jd, float gamma,
                                                     float* __restrict__ ev_out,
                                                     float* __restrict__ dist_out,
                                                     float* __restrict__ coef_out, int E) {
  __shared__ float sc[256 * 35];  // odd row stride: conflict-free per-thread rows
  __shared__ float sv[256 * 3];
  const int64_t eb = (int64_t)blockIdx.x * 256;
  const int nv = (int)min((int64_t)256, (int64_t)E - eb);
  const int t = threadIdx.x;
  if (t < nv) {
    const int64_t e = eb + t;
    const int s = src[e], g = tgt[e];
    float ev[3];
    for (int k = 0; k < 3; ++k) {
      ev[k] = pos[s * 3 + k] - pos[g * 3 + k];
      if (shift) ev[k] = ev[k] + shift[e * 3 + k];
      sv[t * 3 + k] = ev[k];
    }
    dist_out[e] = sqrtf(ev[0] * ev[0] + ev[1] * ev[1] + ev[2] * ev[2]);
    float jl[35];
    for (int k = 0; k < 35; ++k) jl[k] = jd[k];
    float c[35];
    tta_geo::wigner_coef(ev, gamma, jl, c);
    for (int k = 0; k < 35; ++k) sc[t * 35 + k] = c[k];
  }
  __syncthreads();
  for (int i = t; i < nv * 35; i += 256) coef_out[eb * 35 + i] = sc[i];
  for (int i = t; i < nv * 3; i += 256) ev_out[eb * 3 + i] = sv[i];
}

// x_edge[e] = [exp(coeff (d - off_k)^2) (nb) | src_emb[z_src] (ec) | tgt_emb[z_tgt] (ec)], env[e].
__global__ __launch_bounds__(256) void k_edge_features(
    const float* __restrict__ dist, const int* __restrict__ zs, const int* __restrict__ zt,
    const float* __restrict__ semb, const float* __restrict__ temb, const float* __restrict__ off,
    float coeff, float cutoff, int nb, int ec, float* __restrict__ x_edge,
    float* __restrict__ env, int E) {
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int width = nb + 2 * ec;
  if (gid >= (int64_t)E * width) return;
  const int64_t e = gid / width;
  const int k = (int)(gid % width);
  const float d = dist[e];
  float v;
  if (k < nb) {
    const float t = d - off[k];
    v = expf(coeff * (t * t));
  } else if (k < nb + ec) {
    v = semb[(int64_t)zs[e] * ec + (k - nb)];
  } else {
    v = temb[(int64_t)zt[e] * ec + (k - nb - ec)];
  }
  x_edge[gid] = v;
  if (k == 0) env[e] = tta_geo::envelope(d, cutoff);
}

// The same row, one wavefront per edge and four consecutive columns per lane and store
// (nb, ec multiples of 4; 16-byte aligned x_edge and embedding rows): no per-element index
// division and whole 16-byte stores.  The same per-element arithmetic as k_edge_features.
typedef float floatx4e __attribute__((ext_vector_type(4)));
__global__ __launch_bounds__(256) void k_edge_features_v4(
    const float* __restrict__ dist, const int* __restrict__ zs, const int* __restrict__ zt,
    const float* __restrict__ semb, const float* __restrict__ temb, const float* __restrict__ off,
    float coeff, float cutoff, int nb, int ec, float* __restrict__ x_edge,
    float* __restrict__ env, int E) {
  const int lane = threadIdx.x & 63;
  const int64_t e = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (e >= E) return;
  const int w4 = (nb + 2 * ec) / 4, nb4 = nb / 4, ec4 = ec / 4;
  const float d = dist[e];
  floatx4e* row = reinterpret_cast<floatx4e*>(x_edge + e * (int64_t)(nb + 2 * ec));
  const int s = ec ? zs[e] : 0, t = ec ? zt[e] : 0;
  for (int q = lane; q < w4; q += 64) {
    floatx4e v;
    if (q < nb4) {
      const floatx4e o = reinterpret_cast<const floatx4e*>(off)[q];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float u = d - o[i];
        v[i] = expf(coeff * (u * u));
      }
    } else if (q < nb4 + ec4) {
      v = reinterpret_cast<const floatx4e*>(semb + (int64_t)s * ec)[q - nb4];
    } else {
      v = reinterpret_cast<const floatx4e*>(temb + (int64_t)t * ec)[q - nb4 - ec4];
    }
    row[q] = v;
  }
  if (lane == 0) env[e] = tta_geo::envelope(d, cutoff);
}

// The two forward kernels above in one pass, 64 edges per 256-thread block.  Wave 0 forms the
// block's edge vectors and distances (one lane per edge, into LDS with the edges' species), then
// the Wigner coefficients, while waves 1-3 write the block's feature rows with the arithmetic of
// k_edge_features_v4.  The rows of 64 consecutive edges are one contiguous range, taken as a flat
// sequence of float4 columns over the 192 threads, so the stores are contiguous across the waves
// and every thread has independent columns in flight.  The serial Wigner evaluation overlaps the
// row stores instead of running as a launch of its own with one wavefront per SIMD.  Coefficient
// rows and edge vectors leave through LDS with consecutive lanes on consecutive floats.
// Requires the v4 conditions of k_edge_features_v4 and (nb + 2 ec) / 4 < 2^12.
__global__ __launch_bounds__(256) void k_edge_geometry_fwd(
    const float* __restrict__ pos, const int* __restrict__ src, const int* __restrict__ tgt,
    const float* __restrict__ shift, const float* __restrict__ jd, float gamma,
    const int* __restrict__ zs, const int* __restrict__ zt, const float* __restrict__ semb,
    const float* __restrict__ temb, const float* __restrict__ off, float coeff, float cutoff,
    int nb, int ec, float* __restrict__ ev_out, float* __restrict__ dist_out,
    float* __restrict__ coef_out, float* __restrict__ x_edge, float* __restrict__ env, int E) {
  __shared__ float sc[64 * 35];
  __shared__ float sv[64 * 3];
  __shared__ float sd[64];
  __shared__ int sz[2][64];
  const int64_t eb = (int64_t)blockIdx.x * 64;
  const int nv = (int)min((int64_t)64, (int64_t)E - eb);
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  float ev[3] = {0.f, 0.f, 0.f};
  if (w == 0 && lane < nv) {
    const int64_t e = eb + lane;
    const int s = src[e], g = tgt[e];
    for (int k = 0; k < 3; ++k) {
      ev[k] = pos[s * 3 + k] - pos[g * 3 + k];
      if (shift) ev[k] = ev[k] + shift[e * 3 + k];
      sv[lane * 3 + k] = ev[k];
    }
    const float d = sqrtf(ev[0] * ev[0] + ev[1] * ev[1] + ev[2] * ev[2]);
    sd[lane] = d;
    sz[0][lane] = ec ? zs[e] : 0;
    sz[1][lane] = ec ? zt[e] : 0;
    dist_out[e] = d;
    env[e] = tta_geo::envelope(d, cutoff);
  }
  __syncthreads();
  if (w == 0) {
    if (lane < nv) {
      float jl[35];
      for (int k = 0; k < 35; ++k) jl[k] = jd[k];
      float c[35];
      tta_geo::wigner_coef(ev, gamma, jl, c);
      for (int k = 0; k < 35; ++k) sc[lane * 35 + k] = c[k];
    }
  } else {
    const int w4 = (nb + 2 * ec) / 4, nb4 = nb / 4, ec4 = ec / 4;
    const float rw4 = 1.f / (float)w4;
    floatx4e* rows = reinterpret_cast<floatx4e*>(x_edge + eb * (int64_t)(nb + 2 * ec));
    const int total = nv * w4;
#pragma unroll 4
    for (int idx = (int)threadIdx.x - 64; idx < total; idx += 192) {
      // idx / w4 from the float reciprocal (idx < 2^18), corrected to the exact quotient
      int i = (int)((float)idx * rw4);
      i += (i + 1) * w4 <= idx ? 1 : 0;
      i -= i * w4 > idx ? 1 : 0;
      const int q = idx - i * w4;
      floatx4e v;
      if (q < nb4) {
        const float d = sd[i];
        const floatx4e o = reinterpret_cast<const floatx4e*>(off)[q];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float u = d - o[j];
          v[j] = expf(coeff * (u * u));
        }
      } else if (q < nb4 + ec4) {
        v = reinterpret_cast<const floatx4e*>(semb + (int64_t)sz[0][i] * ec)[q - nb4];
      } else {
        v = reinterpret_cast<const floatx4e*>(temb + (int64_t)sz[1][i] * ec)[q - nb4 - ec4];
      }
      rows[idx] = v;
    }
  }
  __syncthreads();
  for (int i = threadIdx.x; i < nv * 35; i += 256) coef_out[eb * 35 + i] = sc[i];
  for (int i = threadIdx.x; i < nv * 3; i += 256) ev_out[eb * 3 + i] = sv[i];
}

// Edge-geometry VJP: g_ev[e] from the adjoints of (coef, gaussians, envelope, |ev|), EPB edges
// per 256-thread block.  The Gaussian-basis adjoint sum_k g[e, k] d/dd exp(coeff (d - off_k)^2)
// runs 16 lanes per edge, each lane a float4 of k per pass (V4: nb and the row stride multiples
// of 4, 16-byte aligned rows; else scalar), so a load instruction covers four edges with 256
// contiguous bytes each; the 16 partial sums reduce by shuffles in a fixed order into LDS.  The
// Wigner-D VJP (geometry_math.h) then runs one thread per edge after the block's barrier and
// reads the edge's coefficient adjoints from LDS, where the block's rows (EPB x 35 contiguous
// floats) arrive by coalesced loads issued before the sums, instead of 35 loads per thread that
// each touch 64 cache lines.  EPB = 256 for graphs large enough to fill the GPU at one thread per
// edge, 64 (the sums over all four waves, the VJP on one) for smaller ones.  Giving the VJP to
// one wave while the other three form the sums measured slower (46 vs 40 us at E = 61,440): the
// sums, not the VJP, bound the kernel.
typedef float floatx4 __attribute__((ext_vector_type(4)));

// This 16-lane group's share of the Gaussian-adjoint sum of edge e, reduced over the group.
template <bool V4>
__device__ __forceinline__ float gauss_adjoint(const float* __restrict__ dist,
                                               const float* __restrict__ g_gauss, int64_t ldg,
                                               const float* __restrict__ off, float coeff, int nb,
                                               int64_t e, bool valid, int sub) {
  float acc = 0.f;
  if (valid) {
    const float d = dist[e];
    const float* gg = g_gauss + e * ldg;
    if (V4) {
      // unrolled so that several rows' loads are in flight before the exponentials
#pragma unroll 8
      for (int k = 4 * sub; k < nb; k += 64) {
        const floatx4 gv = *reinterpret_cast<const floatx4*>(gg + k);
        const floatx4 ov = *reinterpret_cast<const floatx4*>(off + k);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const float t = d - ov[q];
          acc += gv[q] * (expf(coeff * (t * t)) * (coeff * (2.f * t)));
        }
      }
    } else {
      for (int k = sub; k < nb; k += 16) {
        const float t = d - off[k];
        acc += gg[k] * (expf(coeff * (t * t)) * (coeff * (2.f * t)));
      }
    }
  }
  acc += __shfl_xor(acc, 8, 64);
  acc += __shfl_xor(acc, 4, 64);
  acc += __shfl_xor(acc, 2, 64);
  acc += __shfl_xor(acc, 1, 64);
  return acc;
}

template <int EPB, bool V4>
__global__ __launch_bounds__(256) void k_edge_geometry_bwd(
    const float* __restrict__ ev, const float* __restrict__ dist,
    const float* __restrict__ g_coef, const float* __restrict__ g_env,
    const float* __restrict__ g_gauss, int64_t ldg, const float* __restrict__ off, float coeff,
    float cutoff, int nb, const float* __restrict__ jd, float gamma, float* __restrict__ g_ev,
    int E) {
  static_assert(EPB == 64 || EPB == 256, "64 or 256 edges per block");
  __shared__ float sgd[EPB];
  __shared__ float sgc[EPB * 35];  // odd row stride: conflict-free per-thread rows
  const int64_t eb = (int64_t)blockIdx.x * EPB;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, sub = lane & 15, grp = lane >> 4;
  const int nv = (int)min((int64_t)EPB, (int64_t)E - eb);
  const int gclim = nv * 35;
  constexpr int GCL = (EPB * 35 + 255) / 256;  // coalesced g_coef loads per thread
  float gcr[GCL];
  if (g_coef) {
#pragma unroll
    for (int j = 0; j < GCL; ++j)  // every load issued (exact waits), clamped to the block's rows
      gcr[j] = g_coef[eb * 35 + min((int)threadIdx.x + 256 * j, gclim - 1)];
  }
  if (g_gauss) {
#pragma unroll 2
    for (int s = 0; s < EPB / 16; ++s) {
      const int loc = w * (EPB / 4) + s * 4 + grp;  // this 16-lane group's edge in the block
      const float acc =
          gauss_adjoint<V4>(dist, g_gauss, ldg, off, coeff, nb, eb + loc, loc < nv, sub);
      if (sub == 0 && loc < nv) sgd[loc] = acc;
    }
  }
  if (g_coef) {
#pragma unroll
    for (int j = 0; j < GCL; ++j) {
      const int i = (int)threadIdx.x + 256 * j;
      if (i < gclim) sgc[i] = gcr[j];
    }
  }
  __syncthreads();
  const int t = threadIdx.x;
  if (t >= nv) return;
  const int64_t e = eb + t;
  const float v[3] = {ev[e * 3], ev[e * 3 + 1], ev[e * 3 + 2]};
  float out[3] = {0.f, 0.f, 0.f};
  if (g_coef) {
    float jl[35], gc[35];
    for (int k = 0; k < 35; ++k) jl[k] = jd[k];
    for (int k = 0; k < 35; ++k) gc[k] = sgc[t * 35 + k];
    tta_geo::wigner_vjp(v, gamma, jl, gc, out);
  }
  const float d = dist[e];
  float gd = g_gauss ? sgd[t] : 0.f;
  if (g_env) gd += g_env[e] * tta_geo::envelope_grad(d, cutoff);
  if (d > 0.f)
    for (int k = 0; k < 3; ++k) out[k] += gd * (v[k] / d);
  for (int k = 0; k < 3; ++k) g_ev[e * 3 + k] = out[k];
}

// F[n] = -(sum_{src(e) = n} g_ev[e] - sum_{tgt(e) = n} g_ev[e])   (ev = pos[src] - pos[tgt])
// 16 lanes per node: lane j takes the node's source edges j, j + 16, ... and destination edges
// likewise, and the 16 partial sums meet in a fixed xor-tree order (deterministic).
__global__ __launch_bounds__(256) void k_node_forces(const float* __restrict__ g_ev,
                                                     const int* __restrict__ src_ptr,
                                                     const int* __restrict__ src_perm,
                                                     const int* __restrict__ tgt_ptr,
                                                     float* __restrict__ forces, int N) {
  const int gid = blockIdx.x * blockDim.x + threadIdx.x;
  const int n = gid >> 4, j = gid & 15;
  const bool on = n < N;
  float a[3] = {0.f, 0.f, 0.f}, b[3] = {0.f, 0.f, 0.f};
  if (on) {
    for (int k = src_ptr[n] + j; k < src_ptr[n + 1]; k += 16) {
      const int64_t e = src_perm[k];
#pragma unroll
      for (int c = 0; c < 3; ++c) a[c] += g_ev[e * 3 + c];
    }
    for (int64_t e = tgt_ptr[n] + j; e < tgt_ptr[n + 1]; e += 16)
#pragma unroll
      for (int c = 0; c < 3; ++c) b[c] += g_ev[e * 3 + c];
  }
  // every lane of the wavefront takes part in the shuffles (nodes past N contribute zeros)
#pragma unroll
  for (int m = 8; m >= 1; m >>= 1)
#pragma unroll
    for (int c = 0; c < 3; ++c) {
      a[c] += __shfl_xor(a[c], m, 16);
      b[c] += __shfl_xor(b[c], m, 16);
    }
  if (on && j == 0)
    for (int c = 0; c < 3; ++c) forces[(int64_t)n * 3 + c] = -(a[c] - b[c]);
}

// Virial dE/dstrain = sum_e 0.5 (ev_a g_b + ev_b g_a): fixed-order two-stage reduction.
constexpr int kVirBlocks = 256;

__global__ __launch_bounds__(256) void k_virial_partial(const float* __restrict__ ev,
                                                        const float* __restrict__ g_ev, int E,
                                                        float* __restrict__ part) {
  __shared__ float sh[4][9];
  float acc[9];
  for (int i = 0; i < 9; ++i) acc[i] = 0.f;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < E;
       e += (int64_t)gridDim.x * blockDim.x) {
    for (int a = 0; a < 3; ++a)
      for (int b = 0; b < 3; ++b)
        acc[a * 3 + b] += 0.5f * (ev[e * 3 + a] * g_ev[e * 3 + b] + ev[e * 3 + b] * g_ev[e * 3 + a]);
  }
  for (int i = 0; i < 9; ++i) acc[i] = tta_group_sum(acc[i], 64);
  if ((threadIdx.x & 63) == 0)
    for (int i = 0; i < 9; ++i) sh[threadIdx.x >> 6][i] = acc[i];
  __syncthreads();
  if (threadIdx.x < 9) {
    float s = 0.f;
    for (int w = 0; w < 4; ++w) s += sh[w][threadIdx.x];
    part[blockIdx.x * 9 + threadIdx.x] = s;
  }
}

__global__ __launch_bounds__(64) void k_virial_final(const float* __restrict__ part, int nb,
                                                     float* __restrict__ out) {
  const int i = threadIdx.x;
  if (i >= 9) return;
  float s = 0.f;
  for (int b = 0; b < nb; ++b) s += part[b * 9 + i];
  out[i] = s;
}

}  // namespace

// ---------------------------------------------------------------------------------------------
// Allocation-free virial: the partial sums of the two-stage reduction live in this file-scope
// device array instead of a caller workspace.  Every GPU that runs tta_virial_noalloc holds its
// own copy until the process ends.  Host code never passes `scratch` itself (its host-side name
// is not a device address); it passes the per-device address hipGetSymbolAddress returns.
static __device__ __align__(256) float scratch[kVirBlocks * 9];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
float* g_scratch_ptr[kMaxDevices] = {};

// Device address of `scratch` on the current device, resolved once per device (with that
// device current) and kept.
int scratch_for_current_device(const char* who, float** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    tta::set_error("%s: no usable current HIP device (%d)", who, dev);
    return tta::kUnsupported;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr) {
      tta::set_error("%s: hipGetSymbolAddress(scratch) failed on device %d: %s", who, dev,
                     hipGetErrorString(e));
      return tta::kLaunchFailed;
    }
    g_scratch_ptr[dev] = static_cast<float*>(p);
  }
  *out = g_scratch_ptr[dev];
  return tta::kOk;
}

}  // namespace

// Called by tta_check_device (the library's set-up call) for the device it checks.
int tta_init_scratch_current_device() {
  float* p = nullptr;
  return scratch_for_current_device("tta_check_device", &p);
}

extern "C" int tta_edge_wigner(const float* pos, const int* src, const int* tgt,
                               const float* shift, const float* jd, float gamma, float* ev,
                               float* dist, float* coef, int64_t N, int64_t E,
                               hipStream_t stream) {
  TTA_CHECK_ARG(E >= 0 && E < (1ll << 31) && N >= 0, "tta_edge_wigner: bad sizes");
  if (E == 0) return tta::kOk;
  TTA_CHECK_ARG(pos && src && tgt && jd && ev && dist && coef, "tta_edge_wigner: null pointer");
  hipLaunchKernelGGL(k_edge_wigner, dim3(tta_blocks(E, 256)), dim3(256), 0, stream, pos, src, tgt,
                     shift, jd, gamma, ev, dist, coef, (int)E);
  TTA_CHECK_LAUNCH("tta_edge_wigner");
  return tta::kOk;
}

extern "C" int tta_edge_features(const float* dist, const int* zsrc, const int* ztgt,
                                 const float* src_emb, const float* tgt_emb,
                                 const float* offsets, float coeff, float cutoff, int64_t nb,
                                 int64_t ec, float* x_edge, float* env, int64_t E,
                                 hipStream_t stream) {
  TTA_CHECK_ARG(E >= 0 && E < (1ll << 31) && nb > 0 && ec >= 0, "tta_edge_features: bad sizes");
  if (E == 0) return tta::kOk;
  TTA_CHECK_ARG(dist && offsets && x_edge && env && (ec == 0 || (zsrc && ztgt && src_emb && tgt_emb)),
                "tta_edge_features: null pointer");
  const int64_t total = E * (nb + 2 * ec);
  auto al = [](const void* q) { return q == nullptr || ((uintptr_t)q & 15) == 0; };
  if (nb % 4 == 0 && ec % 4 == 0 && al(x_edge) && al(offsets) && al(src_emb) && al(tgt_emb))
    hipLaunchKernelGGL(k_edge_features_v4, dim3(tta_blocks(E, 4)), dim3(256), 0, stream, dist,
                       zsrc, ztgt, src_emb, tgt_emb, offsets, coeff, cutoff, (int)nb, (int)ec,
                       x_edge, env, (int)E);
  else
    hipLaunchKernelGGL(k_edge_features, dim3(tta_blocks(total, 256)), dim3(256), 0, stream,
                       dist, zsrc, ztgt, src_emb, tgt_emb, offsets, coeff, cutoff, (int)nb,
                       (int)ec, x_edge, env, (int)E);
  TTA_CHECK_LAUNCH("tta_edge_features");
  return tta::kOk;
}

extern "C" int tta_edge_geometry_fwd(const float* pos, const int* src, const int* tgt,
                                     const float* shift, const float* jd, float gamma,
                                     const int* zsrc, const int* ztgt, const float* src_emb,
                                     const float* tgt_emb, const float* offsets, float coeff,
                                     float cutoff, int64_t nb, int64_t ec, float* ev, float* dist,
                                     float* coef, float* x_edge, float* env, int64_t N,
                                     int64_t E, hipStream_t stream) {
  TTA_CHECK_ARG(E >= 0 && E < (1ll << 31) && N >= 0 && nb > 0 && ec >= 0,
                "tta_edge_geometry_fwd: bad sizes");
  if (E == 0) return tta::kOk;
  TTA_CHECK_ARG(pos && src && tgt && jd && ev && dist && coef && offsets && x_edge && env &&
                    (ec == 0 || (zsrc && ztgt && src_emb && tgt_emb)),
                "tta_edge_geometry_fwd: null pointer");
  auto al = [](const void* q) { return q == nullptr || ((uintptr_t)q & 15) == 0; };
  if (!(nb % 4 == 0 && ec % 4 == 0 && nb + 2 * ec < (1 << 14) && al(x_edge) && al(offsets) &&
        al(src_emb) && al(tgt_emb))) {
    // rows that the four-column kernel cannot take: the two passes, same arithmetic
    const int st = tta_edge_wigner(pos, src, tgt, shift, jd, gamma, ev, dist, coef, N, E, stream);
    if (st != tta::kOk) return st;
    return tta_edge_features(dist, zsrc, ztgt, src_emb, tgt_emb, offsets, coeff, cutoff, nb, ec,
                             x_edge, env, E, stream);
  }
  hipLaunchKernelGGL(k_edge_geometry_fwd, dim3(tta_blocks(E, 64)), dim3(256), 0, stream, pos, src,
                     tgt, shift, jd, gamma, zsrc, ztgt, src_emb, tgt_emb, offsets, coeff, cutoff,
                     (int)nb, (int)ec, ev, dist, coef, x_edge, env, (int)E);
  TTA_CHECK_LAUNCH("tta_edge_geometry_fwd");
  return tta::kOk;
}

extern "C" int tta_edge_geometry_bwd(const float* ev, const float* dist, const float* g_coef,
                                     const float* g_env, const float* g_gauss, int64_t ldg,
                                     const float* offsets, float coeff, float cutoff, int64_t nb,
                                     const float* jd, float gamma, float* g_ev, int64_t E,
                                     hipStream_t stream) {
  TTA_CHECK_ARG(E >= 0 && E < (1ll << 31), "tta_edge_geometry_bwd: bad sizes");
  if (E == 0) return tta::kOk;
  TTA_CHECK_ARG(ev && dist && jd && g_ev, "tta_edge_geometry_bwd: null pointer");
  TTA_CHECK_ARG(!g_gauss || (offsets && ldg >= nb), "tta_edge_geometry_bwd: bad gaussian adjoint");
  // 256 edges per block (a full thread per edge in phase 2) once there are enough blocks to fill
  // the GPU; small graphs take 64 per block for four times the blocks
  const bool v4 = g_gauss && nb % 4 == 0 && ldg % 4 == 0 && (uintptr_t)g_gauss % 16 == 0 &&
                  (uintptr_t)offsets % 16 == 0;
  const bool wide = E >= 256 * 512;
  auto launch = [&](auto kern, int epb) {
    hipLaunchKernelGGL(kern, dim3(tta_blocks(E, epb)), dim3(256), 0, stream, ev, dist, g_coef,
                       g_env, g_gauss, ldg, offsets, coeff, cutoff, (int)nb, jd, gamma, g_ev,
                       (int)E);
  };
  if (wide)
    v4 ? launch(k_edge_geometry_bwd<256, true>, 256) : launch(k_edge_geometry_bwd<256, false>, 256);
  else
    v4 ? launch(k_edge_geometry_bwd<64, true>, 64) : launch(k_edge_geometry_bwd<64, false>, 64);
  TTA_CHECK_LAUNCH("tta_edge_geometry_bwd");
  return tta::kOk;
}

extern "C" int tta_node_forces(const float* g_ev, const int* src_ptr, const int* src_perm,
                               const int* tgt_ptr, float* forces, int64_t N, int64_t E,
                               hipStream_t stream) {
  TTA_CHECK_ARG(N >= 0 && N < (1ll << 27) && E >= 0, "tta_node_forces: bad sizes (N < 2^27)");
  if (N == 0) return tta::kOk;
  TTA_CHECK_ARG(src_ptr && src_perm && tgt_ptr && forces && (g_ev || E == 0),
                "tta_node_forces: null pointer");
  hipLaunchKernelGGL(k_node_forces, dim3(tta_blocks(N * 16, 256)), dim3(256), 0, stream, g_ev, src_ptr,
                     src_perm, tgt_ptr, forces, (int)N);
  TTA_CHECK_LAUNCH("tta_node_forces");
  return tta::kOk;
}

// `work` must hold kVirBlocks * 9 = 256 * 9 floats.
extern "C" int tta_virial(const float* ev, const float* g_ev, int64_t E, float* work, float* out,
                          hipStream_t stream) {
  TTA_CHECK_ARG(E >= 0 && E < (1ll << 31), "tta_virial: bad sizes");
  TTA_CHECK_ARG(work && out && ((ev && g_ev) || E == 0), "tta_virial: null pointer");
  hipLaunchKernelGGL(k_virial_partial, dim3(kVirBlocks), dim3(256), 0, stream, ev, g_ev, (int)E,
                     work);
  hipLaunchKernelGGL(k_virial_final, dim3(1), dim3(64), 0, stream, work, kVirBlocks, out);
  TTA_CHECK_LAUNCH("tta_virial");
  return tta::kOk;
}

// tta_virial without the workspace argument: the kVirBlocks x 9 partial sums go to this
// device's `scratch`.  Each block writes its whole row, so nothing needs clearing between calls;
// calls that overlap on one GPU (concurrent streams) share the array and race.
extern "C" int tta_virial_noalloc(const float* ev, const float* g_ev, int64_t E, float* out,
                                  hipStream_t stream) {
  TTA_CHECK_ARG(E >= 0 && E < (1ll << 31),
                "tta_virial_noalloc: E = %lld edges is outside [0, 2^31 - 1]", (long long)E);
  TTA_CHECK_ARG(out && ((ev && g_ev) || E == 0), "tta_virial_noalloc: null pointer");
  float* part = nullptr;
  const int st = scratch_for_current_device("tta_virial_noalloc", &part);
  if (st != tta::kOk) return st;
  hipLaunchKernelGGL(k_virial_partial, dim3(kVirBlocks), dim3(256), 0, stream, ev, g_ev, (int)E,
                     part);
  hipLaunchKernelGGL(k_virial_final, dim3(1), dim3(64), 0, stream, part, kVirBlocks, out);
  TTA_CHECK_LAUNCH("tta_virial_noalloc");
  return tta::kOk;
}
