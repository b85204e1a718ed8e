// Radius graph on the GPU, edge for edge and bit for bit equal to the host neighbour list
// (tt_atom.geometry.radius_graph, which restates the reference's geometry.py:48-81 plus the
// per-receiver max-neighbour cap).
//
// Arithmetic (matching the host's torch-CPU fp32 evaluation, checked on the host):
//  * aperiodic: d = ||pos_i - pos_j|| with torch's fp32 norm, which is sqrt(fma(z, z, fma(y, y,
//    x*x))) rounded once; the test d < cutoff (cutoff rounded to fp32) is evaluated without a
//    square root as  s < m^2  in double, m the midpoint between cutoff and its fp32 predecessor
//    (round-to-nearest sqrt(s) < cutoff  <=>  sqrt(s) < m; equality cannot occur for an fp32 s),
//    and d > 0 as s > 0.  Edge (src = i, tgt = j), rows = i, columns j ascending.
//  * periodic: disp = pos_t - (pos_j + shift_c), d2 = (dx*dx + dy*dy) + dz*dz with each product and
//    sum rounded (the host's (disp**2).sum(-1)), kept if min2 < d2 <= cut2.  Edge (src = j,
//    tgt = t, cell c), rows = receivers t, columns (j, c) in lexicographic order.
//  * cap (k > 0): each receiver keeps its k smallest keys (d2, src, cell), d2 of
//    ev = (pos_src - pos_tgt) + shift as ((ex*ex + ey*ey) + ez*ez); the kept edges keep the
//    uncapped order.
// Three passes of one wavefront per row: thresholds (the k-th smallest key of every receiver,
// only with a cap), per-row counts, and the ordered write at the caller's exclusive row offsets.
// Rows of a batch of disjoint systems scan only their own node range [lo, hi).
#include "nl_math.h"

namespace {

using namespace tta_nl;

constexpr int WAVES = 4;
constexpr int MAXC = 1024;  // candidates per receiver held in LDS by the threshold pass

struct NL {
  const float* pos;
  int N;
  const int* lo;  // per-row first candidate node (null: 0)
  const int* hi;  // per-row end (null: N)
  const float* shifts;
  int n_cells;
  const int* clo;  // periodic: per-row first image shift (null: 0); a batch of periodic systems
  const int* chi;  // concatenates their shift tables, each row using its system's (null: n_cells)
  int periodic;
  double mid2;     // aperiodic: keep iff 0 < s < mid2
  float cut2, min2;  // periodic: keep iff min2 < d2 <= cut2
};

// One candidate (column) of a row: periodic rows loop over cells inside the lane.
// Visits, in order, every kept (src, tgt, cell, cap-d2) of row r within column chunk [j0, j0+64).
template <typename F>
__device__ __forceinline__ void row_chunk(const NL& p, int r, int j, float3 pr, F&& f) {
  const float3 pj = ld3(p.pos, j);
  if (!p.periodic) {
    const float s = norm2_fma(pr, pj);
    if (s > 0.f && (double)s < p.mid2) f(r, j, 0, cap_d2(pr, pj, make_float3(0.f, 0.f, 0.f)));
  } else {
    const int c0 = p.clo ? p.clo[r] : 0, c1 = p.chi ? p.chi[r] : p.n_cells;
    for (int c = c0; c < c1; ++c) {
      const float3 sh = ld3(p.shifts, c);
      const float d2 = disp2(pr, pj, sh);
      if (d2 <= p.cut2 && d2 > p.min2) f(j, r, c, cap_d2(pj, pr, sh));
    }
  }
}

// Pass 1 (cap only): k-th smallest key of every receiver t.  Aperiodic candidates are the sources
// i with mask(i, t), keyed (cap_d2(pos_i - pos_t), i, 0); periodic ones are row t's own entries.
__global__ __launch_bounds__(256) void k_nl_thresh(NL p, int k, float* __restrict__ thr_d,
                                                   int* __restrict__ thr_a, int* __restrict__ thr_c,
                                                   int* __restrict__ err) {
  __shared__ float sd[WAVES][MAXC];
  __shared__ int sa[WAVES][MAXC], sc[WAVES][MAXC];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int t = blockIdx.x * WAVES + w;
  if (t >= p.N) return;
  const int lo = p.lo ? p.lo[t] : 0, hi = p.hi ? p.hi[t] : p.N;
  const float3 pt = ld3(p.pos, t);
  int cnt = 0;
  bool overflow = false;
  for (int j0 = lo; j0 < hi; j0 += 64) {
    const int j = j0 + lane;
    int nh = 0;
    float hd[1];
    int ha[1];
    // aperiodic: at most one hit per lane; periodic: up to n_cells, appended by a scan
    if (!p.periodic) {
      if (j < hi) {
        const float3 pi = ld3(p.pos, j);
        const float s = norm2_fma(pi, pt);
        if (s > 0.f && (double)s < p.mid2) {
          nh = 1;
          hd[0] = cap_d2(pi, pt, make_float3(0.f, 0.f, 0.f));
          ha[0] = j;
        }
      }
      int tot;
      const int off = wave_excl_scan(nh, lane, &tot);
      if (nh && cnt + off < MAXC) {
        sd[w][cnt + off] = hd[0];
        sa[w][cnt + off] = ha[0];
        sc[w][cnt + off] = 0;
      }
      cnt += tot;
    } else {
      const float3 pj = j < hi ? ld3(p.pos, j) : make_float3(0.f, 0.f, 0.f);
      const int c0 = p.clo ? p.clo[t] : 0, c1 = p.chi ? p.chi[t] : p.n_cells;
      if (j < hi)
        for (int c = c0; c < c1; ++c) {
          const float d2 = disp2(pt, pj, ld3(p.shifts, c));
          nh += (d2 <= p.cut2 && d2 > p.min2);
        }
      int tot;
      int off = wave_excl_scan(nh, lane, &tot);
      if (nh)
        for (int c = c0; c < c1; ++c) {
          const float3 sh = ld3(p.shifts, c);
          const float d2 = disp2(pt, pj, sh);
          if (d2 <= p.cut2 && d2 > p.min2) {
            if (cnt + off < MAXC) {
              sd[w][cnt + off] = cap_d2(pj, pt, sh);
              sa[w][cnt + off] = j;
              sc[w][cnt + off] = c;
            }
            ++off;
          }
        }
      cnt += tot;
    }
    if (cnt > MAXC) overflow = true;
  }
  if (overflow) {
    if (lane == 0) err[0] = 1;
    return;
  }
  __builtin_amdgcn_wave_barrier();
  if (cnt <= k) {
    if (lane == 0) {
      thr_d[t] = __builtin_inff();
      thr_a[t] = 0x7fffffff;
      thr_c[t] = 0x7fffffff;
    }
    return;
  }
  for (int m = lane; m < cnt; m += 64) {
    const float d = sd[w][m];
    const int a = sa[w][m], c = sc[w][m];
    int rank = 0;
    for (int q = 0; q < cnt; ++q) rank += key_lt(sd[w][q], sa[w][q], sc[w][q], d, a, c);
    if (rank == k - 1) {
      thr_d[t] = d;
      thr_a[t] = a;
      thr_c[t] = c;
    }
  }
}

// Passes 2 and 3: count, then write, the kept entries of every row in order.
template <bool WRITE>
__global__ __launch_bounds__(256) void k_nl_rows(NL p, int cap, const float* __restrict__ thr_d,
                                                 const int* __restrict__ thr_a,
                                                 const int* __restrict__ thr_c,
                                                 int* __restrict__ counts,
                                                 const int64_t* __restrict__ offsets,
                                                 int64_t* __restrict__ e_src,
                                                 int64_t* __restrict__ e_tgt,
                                                 int* __restrict__ e_cell) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int r = blockIdx.x * WAVES + w;
  if (r >= p.N) return;
  const int lo = p.lo ? p.lo[r] : 0, hi = p.hi ? p.hi[r] : p.N;
  const float3 pr = ld3(p.pos, r);
  int64_t base = WRITE ? offsets[r] : 0;
  int total = 0;
  for (int j0 = lo; j0 < hi; j0 += 64) {
    const int j = j0 + lane;
    int nh = 0;
    auto keep = [&](int s, int t, int c, float d2) {
      return !cap || key_le(d2, s, c, thr_d[t], thr_a[t], thr_c[t]);
    };
    if (j < hi)
      row_chunk(p, r, j, pr, [&](int s, int t, int c, float d2) { nh += keep(s, t, c, d2); });
    int tot;
    const int off = wave_excl_scan(nh, lane, &tot);
    if (WRITE && nh) {
      int64_t o = base + off;
      row_chunk(p, r, j, pr, [&](int s, int t, int c, float d2) {
        if (keep(s, t, c, d2)) {
          e_src[o] = s;
          e_tgt[o] = t;
          if (e_cell) e_cell[o] = c;
          ++o;
        }
      });
    }
    base += tot;
    total += tot;
  }
  if (!WRITE && lane == 0) counts[r] = total;
}

}  // namespace

static int check_nl(const float* pos, int64_t N, const float* shifts, int64_t n_cells,
                    const int* clo, const int* chi, int periodic, const char* who) {
  TTA_CHECK_ARG(N >= 0 && N < (1ll << 30), "%s: bad node count", who);
  TTA_CHECK_ARG(N == 0 || pos, "%s: null positions", who);
  TTA_CHECK_ARG(!periodic || (shifts && n_cells > 0 && n_cells < (1 << 20)),
                "%s: periodic graph needs the image-shift table", who);
  TTA_CHECK_ARG((clo == nullptr) == (chi == nullptr), "%s: cell ranges both or neither", who);
  return tta::kOk;
}

static NL make_nl(const float* pos, int64_t N, const int* lo, const int* hi, const float* shifts,
                  int64_t n_cells, const int* clo, const int* chi, int periodic, double mid2,
                  float cut2, float min2) {
  NL p;
  p.pos = pos;
  p.N = (int)N;
  p.lo = lo;
  p.hi = hi;
  p.shifts = shifts;
  p.n_cells = periodic ? (int)n_cells : 1;
  p.clo = periodic ? clo : nullptr;
  p.chi = periodic ? chi : nullptr;
  p.periodic = periodic;
  p.mid2 = mid2;
  p.cut2 = cut2;
  p.min2 = min2;
  return p;
}

extern "C" int tta_radius_graph_thresholds(const float* pos, int64_t N, const int* lo,
                                           const int* hi, const float* shifts, int64_t n_cells,
                                           const int* clo, const int* chi, int periodic, double mid2, float cut2, float min2,
                                           int k, float* thr_d2, int* thr_src, int* thr_cell,
                                           int* err, hipStream_t stream) {
  if (int st = check_nl(pos, N, shifts, n_cells, clo, chi, periodic, "tta_radius_graph_thresholds"))
    return st;
  TTA_CHECK_ARG(k > 0, "tta_radius_graph_thresholds: cap k must be positive");
  TTA_CHECK_ARG(N == 0 || (thr_d2 && thr_src && thr_cell && err),
                "tta_radius_graph_thresholds: null output");
  if (N == 0) return tta::kOk;
  const NL p = make_nl(pos, N, lo, hi, shifts, n_cells, clo, chi, periodic, mid2, cut2, min2);
  hipLaunchKernelGGL(k_nl_thresh, dim3(tta_blocks(N, WAVES)), dim3(64 * WAVES), 0, stream, p, k,
                     thr_d2, thr_src, thr_cell, err);
  TTA_CHECK_LAUNCH("tta_radius_graph_thresholds");
  return tta::kOk;
}

extern "C" int tta_radius_graph_count(const float* pos, int64_t N, const int* lo, const int* hi,
                                      const float* shifts, int64_t n_cells, const int* clo,
                                      const int* chi, int periodic,
                                      double mid2, float cut2, float min2, const float* thr_d2,
                                      const int* thr_src, const int* thr_cell, int* counts,
                                      hipStream_t stream) {
  if (int st = check_nl(pos, N, shifts, n_cells, clo, chi, periodic, "tta_radius_graph_count")) return st;
  TTA_CHECK_ARG(N == 0 || counts, "tta_radius_graph_count: null counts");
  TTA_CHECK_ARG((thr_d2 && thr_src && thr_cell) || (!thr_d2 && !thr_src && !thr_cell),
                "tta_radius_graph_count: thresholds all or none");
  if (N == 0) return tta::kOk;
  const NL p = make_nl(pos, N, lo, hi, shifts, n_cells, clo, chi, periodic, mid2, cut2, min2);
  hipLaunchKernelGGL(k_nl_rows<false>, dim3(tta_blocks(N, WAVES)), dim3(64 * WAVES), 0, stream,
                     p, thr_d2 != nullptr, thr_d2, thr_src, thr_cell, counts, nullptr, nullptr,
                     nullptr, nullptr);
  TTA_CHECK_LAUNCH("tta_radius_graph_count");
  return tta::kOk;
}

extern "C" int tta_radius_graph_write(const float* pos, int64_t N, const int* lo, const int* hi,
                                      const float* shifts, int64_t n_cells, const int* clo,
                                      const int* chi, int periodic,
                                      double mid2, float cut2, float min2, const float* thr_d2,
                                      const int* thr_src, const int* thr_cell,
                                      const int64_t* offsets, int64_t* edge_src,
                                      int64_t* edge_tgt, int* edge_cell, hipStream_t stream) {
  if (int st = check_nl(pos, N, shifts, n_cells, clo, chi, periodic, "tta_radius_graph_write")) return st;
  TTA_CHECK_ARG(N == 0 || (offsets && edge_src && edge_tgt && (!periodic || edge_cell)),
                "tta_radius_graph_write: null output");
  TTA_CHECK_ARG((thr_d2 && thr_src && thr_cell) || (!thr_d2 && !thr_src && !thr_cell),
                "tta_radius_graph_write: thresholds all or none");
  if (N == 0) return tta::kOk;
  const NL p = make_nl(pos, N, lo, hi, shifts, n_cells, clo, chi, periodic, mid2, cut2, min2);
  hipLaunchKernelGGL(k_nl_rows<true>, dim3(tta_blocks(N, WAVES)), dim3(64 * WAVES), 0, stream, p,
                     thr_d2 != nullptr, thr_d2, thr_src, thr_cell, nullptr, offsets, edge_src,
                     edge_tgt, periodic ? edge_cell : nullptr);
  TTA_CHECK_LAUNCH("tta_radius_graph_write");
  return tta::kOk;
}
