// Cell-list radius graph: the same edges, order, image cells and cap as the row-scan list in
// neighbors.hip (and so as the host list, tt_atom.geometry.radius_graph, which restates the
// reference's geometry.py:48-81 plus the per-receiver cap), at O(N) cost instead of O(N^2).
//
// Points.  Every candidate is an image point q = pos_j (+ shift_c) with id = j (aperiodic) or
// id = j * n_cells + c (periodic), so ascending ids are the row-scan column order (j, then c).
// q is rounded exactly as the distance test rounds pos_j + shift_c, so the mask evaluated on q is
// the row scan's mask bit for bit.
//
// Grid.  Bins of side h = 1 / inv_h; bin coordinate u = fl(fl(x - origin) * inv_h).  If a row
// atom p and a point q pass the fp32 distance test, their true distance exceeds the cutoff by
// at most a few ulps of the coordinates, and each computed u is within a few ulps of its exact
// value; the host picks h = cutoff + a margin far above both errors, so |u_p - u_q| < 1 + margin
// on every axis and q lies in one of the 27 bins around p's bin.  Points whose bin falls outside
// the grid are more than h from every row atom (the grid spans the row atoms' bounding box plus
// a bin on every side) and are dropped; row atoms always fall inside it.
//
// Build: count points per bin (atomic slot per point), exclusive scan, scatter the points into
// bin order as float4 (xyz = q, w = id bits).  Within a bin the order is arbitrary: no result
// depends on it (the write pass sorts every row by id; the cap threshold is an exact selection).
//
// Rows (one wavefront each, scanning the 9 contiguous x-runs of the 27 bins around the row atom):
//  * thresholds (cap k only): the k-th smallest key (d2, id) of every receiver, kept by a
//    streaming selection: a sorted buffer of the k smallest keys so far in LDS; every 64
//    candidates below the buffer's current k-th key are sorted across the wave and merged in.
//    Needs O(k) LDS whatever the number of candidates.
//  * count: kept entries per row;
//  * write: the row's kept ids gathered in LDS, sorted (bitonic), written at the caller's row
//    offsets.  A row with more than kRowMax kept entries is not written (err[0] = 1): the caller
//    writes such a graph with the row-scan write pass, which streams its rows in order.
#include "nl_math.h"

namespace {

using namespace tta_nl;

constexpr int kWaves = 4;      // rows per block of the count and write passes
constexpr int kRowMax = 2048;  // kept entries of one row sorted in LDS by the write pass
constexpr int kScanChunk = 2048;  // bins per block of the bin-count scan (256 threads x 8)
constexpr int kMaxK = 1024;    // largest cap of the threshold pass

struct Grid {
  float ox, oy, oz, inv_h;
  int nx, ny, nz;
};

struct CL {
  const float* pos;
  int N;
  const float* shifts;
  int n_cells;
  int periodic;
  Grid g;
  const int* bin_start;  // [nbins + 1]
  const float4* pts;     // binned image points
  double mid2;           // aperiodic: keep iff 0 < s < mid2
  float cut2, min2;      // periodic: keep iff min2 < d2 <= cut2
};

__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__device__ __forceinline__ float bin_u(float x, float o, float inv_h) {
  return rn_mul(rn_sub(x, o), inv_h);
}

// Linear bin of an image point, -1 outside the grid (NaN coordinates included).
__device__ __forceinline__ int point_bin(const Grid& g, float3 q) {
  const float u = bin_u(q.x, g.ox, g.inv_h), v = bin_u(q.y, g.oy, g.inv_h),
              w = bin_u(q.z, g.oz, g.inv_h);
  if (!(u >= 0.f && u < (float)g.nx && v >= 0.f && v < (float)g.ny && w >= 0.f &&
        w < (float)g.nz))
    return -1;
  return ((int)w * g.ny + (int)v) * g.nx + (int)u;
}

__device__ __forceinline__ int clamp_bin(float u, int n) {
  return u >= 0.f ? (u < (float)(n - 1) ? (int)u : n - 1) : 0;
}

// Image point of candidate p (p = j * n_cells + c periodic, j aperiodic): pos_j + shift_c rounded
// per component as the periodic distance test rounds it.
__device__ __forceinline__ float3 image_point(const CL& p, int id) {
  if (!p.periodic) return ld3(p.pos, id);
  const int j = id / p.n_cells, c = id - j * p.n_cells;
  const float3 pj = ld3(p.pos, j), sh = ld3(p.shifts, c);
  return make_float3(rn_add(pj.x, sh.x), rn_add(pj.y, sh.y), rn_add(pj.z, sh.z));
}

// Visits every binned point of the 27 bins around row atom pr, 64 per step (wave-uniform loop):
// f(valid, q) per lane.
template <typename F>
__device__ __forceinline__ void for_candidates(const CL& p, float3 pr, int lane, F&& f) {
  const Grid& g = p.g;
  const int bx = clamp_bin(bin_u(pr.x, g.ox, g.inv_h), g.nx);
  const int by = clamp_bin(bin_u(pr.y, g.oy, g.inv_h), g.ny);
  const int bz = clamp_bin(bin_u(pr.z, g.oz, g.inv_h), g.nz);
  const int x0 = max(bx - 1, 0), x1 = min(bx + 1, g.nx - 1);
  for (int z = max(bz - 1, 0); z <= min(bz + 1, g.nz - 1); ++z)
    for (int y = max(by - 1, 0); y <= min(by + 1, g.ny - 1); ++y) {
      const int row = (z * g.ny + y) * g.nx;
      const int s = p.bin_start[row + x0], e = p.bin_start[row + x1 + 1];
      for (int i0 = s; i0 < e; i0 += 64) {
        const int i = i0 + lane;
        const bool ok = i < e;
        f(ok, ok ? p.pts[i] : make_float4(0.f, 0.f, 0.f, 0.f));
      }
    }
}

// Mask of a (row atom, point) pair, evaluated as the row scan evaluates it.
__device__ __forceinline__ bool rows_mask(const CL& p, float3 pr, float4 q) {
  if (!p.periodic) {
    const float s = norm2_fma(pr, make_float3(q.x, q.y, q.z));
    return s > 0.f && (double)s < p.mid2;
  }
  const float d2 = sum_sq(rn_sub(pr.x, q.x), rn_sub(pr.y, q.y), rn_sub(pr.z, q.z));
  return d2 <= p.cut2 && d2 > p.min2;
}

// Cap key distance of the edge between row atom r (at pr) and candidate id (image point q):
// aperiodic rows are sources (edge r -> id), periodic rows receivers (edge (j, c) -> r).
__device__ __forceinline__ float edge_d2(const CL& p, float3 pr, float4 q, int id) {
  if (!p.periodic) return cap_d2(pr, make_float3(q.x, q.y, q.z), make_float3(0.f, 0.f, 0.f));
  const int j = id / p.n_cells, c = id - j * p.n_cells;
  return cap_d2(ld3(p.pos, j), pr, ld3(p.shifts, c));
}

__device__ __forceinline__ bool klt(float d, int a, float D, int A) {
  return d < D || (d == D && a < A);
}

// Ascending bitonic sort of one (d, id) key per lane across the wave.
__device__ __forceinline__ void wave_sort(float& d, int& a, int lane) {
#pragma unroll
  for (int k = 2; k <= 64; k <<= 1)
#pragma unroll
    for (int j = k >> 1; j > 0; j >>= 1) {
      const float od = __shfl_xor(d, j, 64);
      const int oa = __shfl_xor(a, j, 64);
      const bool up = (lane & k) == 0, lower = (lane & j) == 0;
      if (lower == up ? klt(od, oa, d, a) : klt(d, a, od, oa)) {
        d = od;
        a = oa;
      }
    }
}

// ---------------------------------------------------------------------------- build
__global__ __launch_bounds__(256) void k_cl_zero(int* __restrict__ a, int64_t n) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x)
    a[i] = 0;
}

__global__ __launch_bounds__(256) void k_cl_bin(CL p, int64_t P, int* __restrict__ bin_count,
                                                int* __restrict__ pt_bin,
                                                int* __restrict__ pt_slot) {
  const int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (i >= P) return;
  const int b = point_bin(p.g, image_point(p, (int)i));
  pt_bin[i] = b;
  if (b >= 0) pt_slot[i] = atomicAdd(&bin_count[b], 1);
}

// Per-block sums of kScanChunk bin counts.
__global__ __launch_bounds__(256) void k_cl_scan_sums(const int* __restrict__ cnt, int nb,
                                                      int* __restrict__ sums) {
  __shared__ int red[4];
  const int base = blockIdx.x * kScanChunk;
  int s = 0;
  for (int i = threadIdx.x; i < kScanChunk; i += 256)
    if (base + i < nb) s += cnt[base + i];
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o, 64);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = s;
  __syncthreads();
  if (threadIdx.x == 0) sums[blockIdx.x] = red[0] + red[1] + red[2] + red[3];
}

// Exclusive scan of the block sums in place (one block, any count).
__global__ __launch_bounds__(256) void k_cl_scan_top(int* __restrict__ sums, int n) {
  __shared__ int wsum[4];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  int carry = 0;
  for (int b0 = 0; b0 < n; b0 += 256) {
    const int i = b0 + threadIdx.x;
    const int v = i < n ? sums[i] : 0;
    int tot;
    const int ex = wave_excl_scan(v, lane, &tot);
    if (lane == 0) wsum[w] = tot;
    __syncthreads();
    int wo = 0;
    for (int q = 0; q < w; ++q) wo += wsum[q];
    const int all = wsum[0] + wsum[1] + wsum[2] + wsum[3];
    if (i < n) sums[i] = carry + wo + ex;
    carry += all;
    __syncthreads();
  }
}

// bin_start[b] = exclusive prefix of the counts; bin_start[nb] = total.
__global__ __launch_bounds__(256) void k_cl_scan_apply(const int* __restrict__ cnt, int nb,
                                                       const int* __restrict__ sums,
                                                       int* __restrict__ start) {
  __shared__ int wsum[4];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int base = blockIdx.x * kScanChunk + threadIdx.x * 8;
  int v[8], s = 0;
#pragma unroll
  for (int q = 0; q < 8; ++q) {
    v[q] = base + q < nb ? cnt[base + q] : 0;
    s += v[q];
  }
  int tot;
  const int ex = wave_excl_scan(s, lane, &tot);
  if (lane == 0) wsum[w] = tot;
  __syncthreads();
  int run = sums[blockIdx.x] + ex;
  for (int q = 0; q < w; ++q) run += wsum[q];
#pragma unroll
  for (int q = 0; q < 8; ++q) {
    if (base + q < nb) start[base + q] = run;
    run += v[q];
    if (base + q == nb - 1) start[nb] = run;
  }
}

__global__ __launch_bounds__(256) void k_cl_fill(CL p, int64_t P, const int* __restrict__ pt_bin,
                                                 const int* __restrict__ pt_slot,
                                                 float4* __restrict__ pts) {
  const int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (i >= P) return;
  const int b = pt_bin[i];
  if (b < 0) return;
  const float3 q = image_point(p, (int)i);
  pts[p.bin_start[b] + pt_slot[i]] = make_float4(q.x, q.y, q.z, __int_as_float((int)i));
}

// ---------------------------------------------------------------------------- rows
// Thresholds: k-th smallest cap key of every receiver t (sentinel when it has <= k candidates).
// Dynamic LDS per wave: two key buffers of k entries and one 64-entry batch, (float, int) each.
__global__ __launch_bounds__(256) void k_cl_thresh(CL p, int k, float* __restrict__ thr_d,
                                                   int* __restrict__ thr_a,
                                                   int* __restrict__ thr_c) {
  extern __shared__ unsigned char smem[];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, waves = blockDim.x >> 6;
  const int t = blockIdx.x * waves + w;
  if (t >= p.N) return;
  float* bd[2];
  int* ba[2];
  unsigned char* base = smem + (size_t)w * (size_t)(2 * k + 64) * 8;
  bd[0] = (float*)base;
  ba[0] = (int*)(base + 4 * k);
  bd[1] = (float*)(base + 8 * k);
  ba[1] = (int*)(base + 12 * k);
  float* sd = (float*)(base + 16 * k);
  int* sa = (int*)(base + 16 * k + 256);
  const float3 pt = ld3(p.pos, t);
  int m = 0, cur = 0, total = 0;
  float td = __builtin_inff();  // current k-th key (+inf until the buffer holds k keys)
  int ta = 0x7fffffff;
  for_candidates(p, pt, lane, [&](bool ok, float4 q) {
    bool hit = false;
    float d = __builtin_inff();
    int a = 0x7fffffff;
    if (ok) {
      const int id = __float_as_int(q.w);
      const float3 pq = make_float3(q.x, q.y, q.z);
      if (!p.periodic) {
        const float s = norm2_fma(pq, pt);
        hit = s > 0.f && (double)s < p.mid2;
        if (hit) d = cap_d2(pq, pt, make_float3(0.f, 0.f, 0.f));
      } else {
        const float d2 = sum_sq(rn_sub(pt.x, q.x), rn_sub(pt.y, q.y), rn_sub(pt.z, q.z));
        hit = d2 <= p.cut2 && d2 > p.min2;
        if (hit) {
          const int j = id / p.n_cells, c = id - j * p.n_cells;
          d = cap_d2(ld3(p.pos, j), pt, ld3(p.shifts, c));
        }
      }
      if (hit) a = id;
    }
    total += __popcll(__ballot(hit));
    const bool take = hit && klt(d, a, td, ta);
    if (!__ballot(take)) return;
    if (!take) {
      d = __builtin_inff();
      a = 0x7fffffff;
    }
    wave_sort(d, a, lane);
    const int nb = __popcll(__ballot(take));
    sd[lane] = d;
    sa[lane] = a;
    wave_sync();
    float* od = bd[cur];
    int* oa = ba[cur];
    float* nd = bd[cur ^ 1];
    int* na = ba[cur ^ 1];
    for (int b = lane; b < m; b += 64) {
      const float kd = od[b];
      const int ka = oa[b];
      int lo = 0, hi = nb;
      while (lo < hi) {
        const int mid = (lo + hi) >> 1;
        if (klt(sd[mid], sa[mid], kd, ka)) lo = mid + 1; else hi = mid;
      }
      if (b + lo < k) {
        nd[b + lo] = kd;
        na[b + lo] = ka;
      }
    }
    if (lane < nb) {
      int lo = 0, hi = m;
      while (lo < hi) {
        const int mid = (lo + hi) >> 1;
        if (klt(od[mid], oa[mid], d, a)) lo = mid + 1; else hi = mid;
      }
      if (lane + lo < k) {
        nd[lane + lo] = d;
        na[lane + lo] = a;
      }
    }
    wave_sync();
    cur ^= 1;
    m = min(k, m + nb);
    if (m == k) {
      td = bd[cur][k - 1];
      ta = ba[cur][k - 1];
    }
  });
  if (lane == 0) {
    if (total <= k) {
      thr_d[t] = __builtin_inff();
      thr_a[t] = 0x7fffffff;
      thr_c[t] = 0x7fffffff;
    } else {
      thr_d[t] = td;
      thr_a[t] = p.periodic ? ta / p.n_cells : ta;
      thr_c[t] = p.periodic ? ta - (ta / p.n_cells) * p.n_cells : 0;
    }
  }
}

// Is the entry (row r, candidate id) kept by the cap thresholds?
__device__ __forceinline__ bool cap_keep(const CL& p, int r, float3 pr, float4 q, int id,
                                         const float* thr_d, const int* thr_a, const int* thr_c) {
  const float d2 = edge_d2(p, pr, q, id);
  if (!p.periodic) return key_le(d2, r, 0, thr_d[id], thr_a[id], thr_c[id]);
  const int j = id / p.n_cells, c = id - j * p.n_cells;
  return key_le(d2, j, c, thr_d[r], thr_a[r], thr_c[r]);
}

__global__ __launch_bounds__(256) void k_cl_count(CL p, const float* __restrict__ thr_d,
                                                  const int* __restrict__ thr_a,
                                                  const int* __restrict__ thr_c,
                                                  int* __restrict__ counts) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int r = blockIdx.x * kWaves + w;
  if (r >= p.N) return;
  const float3 pr = ld3(p.pos, r);
  int total = 0;
  for_candidates(p, pr, lane, [&](bool ok, float4 q) {
    bool keep = ok && rows_mask(p, pr, q);
    if (keep && thr_d) keep = cap_keep(p, r, pr, q, __float_as_int(q.w), thr_d, thr_a, thr_c);
    total += __popcll(__ballot(keep));
  });
  if (lane == 0) counts[r] = total;
}

__global__ __launch_bounds__(256) void k_cl_write(CL p, const float* __restrict__ thr_d,
                                                  const int* __restrict__ thr_a,
                                                  const int* __restrict__ thr_c,
                                                  const int64_t* __restrict__ offsets,
                                                  int64_t* __restrict__ e_src,
                                                  int64_t* __restrict__ e_tgt,
                                                  int* __restrict__ e_cell, int* __restrict__ err) {
  __shared__ int ids[kWaves][kRowMax];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int r = blockIdx.x * kWaves + w;
  if (r >= p.N) return;
  const float3 pr = ld3(p.pos, r);
  int* s = ids[w];
  int cnt = 0;
  for_candidates(p, pr, lane, [&](bool ok, float4 q) {
    const int id = __float_as_int(q.w);
    bool keep = ok && rows_mask(p, pr, q);
    if (keep && thr_d) keep = cap_keep(p, r, pr, q, id, thr_d, thr_a, thr_c);
    const uint64_t bal = __ballot(keep);
    const int off = __popcll(bal & ((1ull << lane) - 1ull));
    if (keep && cnt + off < kRowMax) s[cnt + off] = id;
    cnt += __popcll(bal);
  });
  if (cnt > kRowMax) {
    if (lane == 0) err[0] = 1;
    return;
  }
  if (cnt == 0) return;
  int n = 64;
  while (n < cnt) n <<= 1;
  for (int i = cnt + lane; i < n; i += 64) s[i] = 0x7fffffff;
  wave_sync();
  for (int k = 2; k <= n; k <<= 1)
    for (int j = k >> 1; j > 0; j >>= 1) {
      for (int t = lane; t < (n >> 1); t += 64) {
        const int lo = ((t & ~(j - 1)) << 1) | (t & (j - 1)), hi = lo + j;
        const int a = s[lo], b = s[hi];
        if ((a > b) == ((lo & k) == 0)) {
          s[lo] = b;
          s[hi] = a;
        }
      }
      wave_sync();
    }
  const int64_t o = offsets[r];
  for (int i = lane; i < cnt; i += 64) {
    const int id = s[i];
    if (!p.periodic) {
      e_src[o + i] = r;
      e_tgt[o + i] = id;
    } else {
      const int j = id / p.n_cells;
      e_src[o + i] = j;
      e_tgt[o + i] = r;
      e_cell[o + i] = id - j * p.n_cells;
    }
  }
}

}  // namespace

static int check_cells(const float* pos, int64_t N, const float* shifts, int64_t n_cells,
                       int periodic, const tta_cell_grid* grid, const char* who) {
  TTA_CHECK_ARG(N >= 0 && N < (1ll << 30), "%s: bad node count", who);
  TTA_CHECK_ARG(N == 0 || pos, "%s: null positions", who);
  TTA_CHECK_ARG(!periodic || (shifts && n_cells > 0 && N * n_cells < (1ll << 30)),
                "%s: periodic points need the image-shift table and N * n_cells < 2^30", who);
  TTA_CHECK_ARG(grid, "%s: null grid", who);
  const int64_t nb = (int64_t)grid->dims[0] * grid->dims[1] * grid->dims[2];
  TTA_CHECK_ARG(grid->dims[0] > 0 && grid->dims[1] > 0 && grid->dims[2] > 0 && nb < (1ll << 28),
                "%s: bad grid dimensions", who);
  TTA_CHECK_ARG(grid->inv_h > 0.f && grid->inv_h < 1e30f, "%s: bad bin size", who);
  return tta::kOk;
}

static CL make_cl(const float* pos, int64_t N, const float* shifts, int64_t n_cells,
                  int periodic, const tta_cell_grid* grid, const int* bin_start,
                  const float* points, double mid2, float cut2, float min2) {
  CL p;
  p.pos = pos;
  p.N = (int)N;
  p.shifts = shifts;
  p.n_cells = periodic ? (int)n_cells : 1;
  p.periodic = periodic;
  p.g.ox = grid->origin[0];
  p.g.oy = grid->origin[1];
  p.g.oz = grid->origin[2];
  p.g.inv_h = grid->inv_h;
  p.g.nx = grid->dims[0];
  p.g.ny = grid->dims[1];
  p.g.nz = grid->dims[2];
  p.bin_start = bin_start;
  p.pts = (const float4*)points;
  p.mid2 = mid2;
  p.cut2 = cut2;
  p.min2 = min2;
  return p;
}

extern "C" int64_t tta_cell_list_workspace(int64_t n_bins, int64_t n_points) {
  return n_bins + 2 * n_points + (n_bins + kScanChunk - 1) / kScanChunk;
}

extern "C" int tta_cell_list_build(const float* pos, int64_t N, const float* shifts,
                                   int64_t n_cells, int periodic, const tta_cell_grid* grid,
                                   int* bin_start, float* points, int* work, hipStream_t stream) {
  if (int st = check_cells(pos, N, shifts, n_cells, periodic, grid, "tta_cell_list_build"))
    return st;
  TTA_CHECK_ARG(bin_start && points && work, "tta_cell_list_build: null output or workspace");
  const int64_t nb = (int64_t)grid->dims[0] * grid->dims[1] * grid->dims[2];
  const int64_t P = periodic ? N * n_cells : N;
  int* bin_count = work;
  int* pt_bin = work + nb;
  int* pt_slot = pt_bin + P;
  int* sums = pt_slot + P;
  const int nsum = (int)((nb + kScanChunk - 1) / kScanChunk);
  const CL p = make_cl(pos, N, shifts, n_cells, periodic, grid, bin_start, points, 0.0, 0.f, 0.f);
  hipLaunchKernelGGL(k_cl_zero, dim3(tta_blocks(nb, 256) < 4096 ? tta_blocks(nb, 256) : 4096u),
                     dim3(256), 0, stream, bin_count, nb);
  if (P) hipLaunchKernelGGL(k_cl_bin, dim3(tta_blocks(P, 256)), dim3(256), 0, stream, p, P,
                            bin_count, pt_bin, pt_slot);
  hipLaunchKernelGGL(k_cl_scan_sums, dim3(nsum), dim3(256), 0, stream, bin_count, (int)nb, sums);
  hipLaunchKernelGGL(k_cl_scan_top, dim3(1), dim3(256), 0, stream, sums, nsum);
  hipLaunchKernelGGL(k_cl_scan_apply, dim3(nsum), dim3(256), 0, stream, bin_count, (int)nb, sums,
                     bin_start);
  if (P) hipLaunchKernelGGL(k_cl_fill, dim3(tta_blocks(P, 256)), dim3(256), 0, stream, p, P,
                            pt_bin, pt_slot, (float4*)points);
  TTA_CHECK_LAUNCH("tta_cell_list_build");
  return tta::kOk;
}

extern "C" int tta_radius_graph_cells_thresholds(const float* pos, int64_t N, const float* shifts,
                                                 int64_t n_cells, int periodic,
                                                 const tta_cell_grid* grid, const int* bin_start,
                                                 const float* points, double mid2, float cut2,
                                                 float min2, int k, float* thr_d2, int* thr_src,
                                                 int* thr_cell, hipStream_t stream) {
  if (int st = check_cells(pos, N, shifts, n_cells, periodic, grid,
                           "tta_radius_graph_cells_thresholds"))
    return st;
  TTA_CHECK_ARG(k > 0 && k <= kMaxK, "tta_radius_graph_cells_thresholds: cap k must be in "
                "[1, %d], got %d", kMaxK, k);
  TTA_CHECK_ARG(N == 0 || (bin_start && points && thr_d2 && thr_src && thr_cell),
                "tta_radius_graph_cells_thresholds: null cell list or output");
  if (N == 0) return tta::kOk;
  const CL p = make_cl(pos, N, shifts, n_cells, periodic, grid, bin_start, points, mid2, cut2,
                       min2);
  const int waves = k <= 256 ? 4 : 1;
  const size_t lds = (size_t)waves * (size_t)(2 * k + 64) * 8;
  hipLaunchKernelGGL(k_cl_thresh, dim3(tta_blocks(N, waves)), dim3(64 * waves), lds, stream, p,
                     k, thr_d2, thr_src, thr_cell);
  TTA_CHECK_LAUNCH("tta_radius_graph_cells_thresholds");
  return tta::kOk;
}

extern "C" int tta_radius_graph_cells_count(const float* pos, int64_t N, const float* shifts,
                                            int64_t n_cells, int periodic,
                                            const tta_cell_grid* grid, const int* bin_start,
                                            const float* points, double mid2, float cut2,
                                            float min2, const float* thr_d2, const int* thr_src,
                                            const int* thr_cell, int* counts,
                                            hipStream_t stream) {
  if (int st = check_cells(pos, N, shifts, n_cells, periodic, grid,
                           "tta_radius_graph_cells_count"))
    return st;
  TTA_CHECK_ARG(N == 0 || (bin_start && points && counts),
                "tta_radius_graph_cells_count: null cell list or counts");
  TTA_CHECK_ARG((thr_d2 && thr_src && thr_cell) || (!thr_d2 && !thr_src && !thr_cell),
                "tta_radius_graph_cells_count: thresholds all or none");
  if (N == 0) return tta::kOk;
  const CL p = make_cl(pos, N, shifts, n_cells, periodic, grid, bin_start, points, mid2, cut2,
                       min2);
  hipLaunchKernelGGL(k_cl_count, dim3(tta_blocks(N, kWaves)), dim3(64 * kWaves), 0, stream, p,
                     thr_d2, thr_src, thr_cell, counts);
  TTA_CHECK_LAUNCH("tta_radius_graph_cells_count");
  return tta::kOk;
}

extern "C" int tta_radius_graph_cells_write(const float* pos, int64_t N, const float* shifts,
                                            int64_t n_cells, int periodic,
                                            const tta_cell_grid* grid, const int* bin_start,
                                            const float* points, double mid2, float cut2,
                                            float min2, const float* thr_d2, const int* thr_src,
                                            const int* thr_cell, const int64_t* offsets,
                                            int64_t* edge_src, int64_t* edge_tgt, int* edge_cell,
                                            int* err, hipStream_t stream) {
  if (int st = check_cells(pos, N, shifts, n_cells, periodic, grid,
                           "tta_radius_graph_cells_write"))
    return st;
  TTA_CHECK_ARG(N == 0 || (bin_start && points && offsets && edge_src && edge_tgt && err &&
                           (!periodic || edge_cell)),
                "tta_radius_graph_cells_write: null cell list or output");
  TTA_CHECK_ARG((thr_d2 && thr_src && thr_cell) || (!thr_d2 && !thr_src && !thr_cell),
                "tta_radius_graph_cells_write: thresholds all or none");
  if (N == 0) return tta::kOk;
  const CL p = make_cl(pos, N, shifts, n_cells, periodic, grid, bin_start, points, mid2, cut2,
                       min2);
  hipLaunchKernelGGL(k_cl_write, dim3(tta_blocks(N, kWaves)), dim3(64 * kWaves), 0, stream, p,
                     thr_d2, thr_src, thr_cell, offsets, edge_src, edge_tgt,
                     periodic ? edge_cell : nullptr, err);
  TTA_CHECK_LAUNCH("tta_radius_graph_cells_write");
  return tta::kOk;
}
