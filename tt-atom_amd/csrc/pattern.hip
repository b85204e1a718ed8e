// Per-op entry points of the reference's rotation and scatter modules, for callers that drive the
// eSCN-MD blocks op by op instead of through the fused step:
//  * a rotation by a per-edge matrix with a fixed sparsity pattern (rotation.py:211-260): the
//    pattern's nnz structural nonzeros (i_k, j_k) are shared by all edges, their values are the
//    packed coefficients coef[e, k];
//  * the edge -> node sum over a fixed-width gather table (scatter.py:62-89).
// The fused step uses the specialised kernels of rotate.hip instead; these serve any pattern
// (rectangular, any lmax), any channel count and the reference's table layout.
#include "common.h"

namespace {

constexpr int kMaxNnz = 512, kMaxRows = 64, kMaxBlocks = 255;

// A pattern grouped by output block: the terms of output block r are q in [ptr[r], ptr[r+1]),
// each coefficient column k[q] times input block blk[q] (kernel arguments: read-only, uniform).
struct RotPattern {
  uint16_t ptr[kMaxRows + 1];
  uint16_t k[kMaxNnz];
  uint8_t blk[kMaxNnz];
};

// out[e, r, w] = sum_q coef[e, k_q] x[e, blk_q, w] over the terms of block r, in pattern order.
// One thread per output element; consecutive threads take consecutive channels.
__global__ __launch_bounds__(256) void k_rotate_pattern(const float* __restrict__ x,
                                                        const float* __restrict__ coef,
                                                        float* __restrict__ out, int64_t E,
                                                        int n_in, int n_out, int W, int nnz,
                                                        RotPattern pat) {
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t per_edge = (int64_t)n_out * W;
  if (gid >= E * per_edge) return;
  const int64_t e = gid / per_edge;
  const int rw = (int)(gid - e * per_edge);
  const int r = rw / W, w = rw - r * W;
  const float* xe = x + e * (int64_t)n_in * W + w;
  const float* ce = coef + e * (int64_t)nnz;
  float acc = 0.f;
  for (int q = pat.ptr[r]; q < pat.ptr[r + 1]; ++q) acc += ce[pat.k[q]] * xe[pat.blk[q] * W];
  out[gid] = acc;
}

// gc[e, k] = sum_w g_out[e, i_k, w] x_in[e, j_k, w]: one wavefront per (edge, nonzero), lanes
// striding over the channels, then a fixed butterfly (deterministic).
struct GcPattern {
  uint8_t i[kMaxNnz];
  uint8_t j[kMaxNnz];
};

__global__ __launch_bounds__(256) void k_rotate_pattern_gc(const float* __restrict__ g_out,
                                                           const float* __restrict__ x_in,
                                                           float* __restrict__ gc, int64_t E,
                                                           int n_in, int n_out, int W, int nnz,
                                                           GcPattern pat) {
  const int64_t wave = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
  const int lane = threadIdx.x & 63;
  if (wave >= E * nnz) return;
  const int64_t e = wave / nnz;
  const int k = (int)(wave - e * nnz);
  const float* go = g_out + (e * n_out + pat.i[k]) * (int64_t)W;
  const float* xi = x_in + (e * n_in + pat.j[k]) * (int64_t)W;
  float acc = 0.f;
  for (int w = lane; w < W; w += 64) acc += go[w] * xi[w];
  acc = tta_group_sum(acc, 64);
  if (lane == 0) gc[wave] = acc;
}

// out[n, w] = sum_d msg[g, w] for g = gather[n * Dmax + d], d = 0 .. Dmax - 1 in order; an index
// outside [0, n_msg) (the table's sentinel: the zero row appended to the messages) adds nothing.
__global__ __launch_bounds__(256) void k_segment_sum_table(const float* __restrict__ msg,
                                                           const int* __restrict__ gather,
                                                           float* __restrict__ out, int64_t N,
                                                           int Dmax, int W, int64_t n_msg) {
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= N * W) return;
  const int64_t n = gid / W;
  const int w = (int)(gid - n * W);
  const int* gr = gather + n * Dmax;
  float acc = 0.f;
  for (int d = 0; d < Dmax; ++d) {
    const int g = gr[d];
    if (g >= 0 && g < n_msg) acc += msg[(int64_t)g * W + w];
  }
  out[gid] = acc;
}

}  // namespace

extern "C" int tta_rotate_pattern(const float* x, const float* coef, float* out, int64_t E,
                                  int64_t n_in, int64_t n_out, int64_t W, int64_t nnz,
                                  const int* ptr, const int* k, const int* blk,
                                  hipStream_t stream) {
  TTA_CHECK_ARG(E >= 0 && W > 0 && n_in > 0 && n_in <= kMaxBlocks && n_out > 0 &&
                    n_out <= kMaxRows && nnz >= 0 && nnz <= kMaxNnz,
                "tta_rotate_pattern: sizes out of range (n_in <= %d, n_out <= %d, nnz <= %d)",
                kMaxBlocks, kMaxRows, kMaxNnz);
  TTA_CHECK_ARG(E * n_out * W < ((int64_t)1 << 40) && n_in * W < (1 << 30),
                "tta_rotate_pattern: tensor too large");
  TTA_CHECK_ARG(ptr && (nnz == 0 || (k && blk)), "tta_rotate_pattern: null pattern");
  RotPattern pat{};
  TTA_CHECK_ARG(ptr[0] == 0 && ptr[n_out] == nnz, "tta_rotate_pattern: ptr must run 0 .. nnz");
  for (int64_t r = 0; r <= n_out; ++r) {
    TTA_CHECK_ARG(r == 0 || ptr[r] >= ptr[r - 1], "tta_rotate_pattern: ptr must not decrease");
    pat.ptr[r] = (uint16_t)ptr[r];
  }
  for (int64_t q = 0; q < nnz; ++q) {
    TTA_CHECK_ARG(k[q] >= 0 && k[q] < nnz && blk[q] >= 0 && blk[q] < n_in,
                  "tta_rotate_pattern: term %lld out of range", (long long)q);
    pat.k[q] = (uint16_t)k[q];
    pat.blk[q] = (uint8_t)blk[q];
  }
  if (E == 0) return tta::kOk;
  TTA_CHECK_ARG(x && out && (coef || nnz == 0), "tta_rotate_pattern: null pointer");
  hipLaunchKernelGGL(k_rotate_pattern, dim3(tta_blocks(E * n_out * W, 256)), dim3(256), 0, stream,
                     x, coef, out, E, (int)n_in, (int)n_out, (int)W, (int)nnz, pat);
  TTA_CHECK_LAUNCH("tta_rotate_pattern");
  return tta::kOk;
}

extern "C" int tta_rotate_pattern_gc(const float* g_out, const float* x_in, float* gc, int64_t E,
                                     int64_t n_in, int64_t n_out, int64_t W, int64_t nnz,
                                     const int* ii, const int* jj, hipStream_t stream) {
  TTA_CHECK_ARG(E >= 0 && W > 0 && n_in > 0 && n_in <= kMaxBlocks && n_out > 0 &&
                    n_out <= kMaxBlocks && nnz >= 0 && nnz <= kMaxNnz,
                "tta_rotate_pattern_gc: sizes out of range (n_in, n_out <= %d, nnz <= %d)",
                kMaxBlocks, kMaxNnz);
  TTA_CHECK_ARG(E * nnz < ((int64_t)1 << 34) && (int64_t)n_in * W < (1 << 30) &&
                    (int64_t)n_out * W < (1 << 30),
                "tta_rotate_pattern_gc: tensor too large");
  TTA_CHECK_ARG(nnz == 0 || (ii && jj), "tta_rotate_pattern_gc: null pattern");
  GcPattern pat{};
  for (int64_t q = 0; q < nnz; ++q) {
    TTA_CHECK_ARG(ii[q] >= 0 && ii[q] < n_out && jj[q] >= 0 && jj[q] < n_in,
                  "tta_rotate_pattern_gc: nonzero %lld out of range", (long long)q);
    pat.i[q] = (uint8_t)ii[q];
    pat.j[q] = (uint8_t)jj[q];
  }
  if (E == 0 || nnz == 0) return tta::kOk;
  TTA_CHECK_ARG(g_out && x_in && gc, "tta_rotate_pattern_gc: null pointer");
  hipLaunchKernelGGL(k_rotate_pattern_gc, dim3(tta_blocks(E * nnz * 64, 256)), dim3(256), 0,
                     stream, g_out, x_in, gc, E, (int)n_in, (int)n_out, (int)W, (int)nnz, pat);
  TTA_CHECK_LAUNCH("tta_rotate_pattern_gc");
  return tta::kOk;
}

extern "C" int tta_segment_sum_table(const float* msg, const int* gather, float* out,
                                     int64_t n_msg, int64_t N, int64_t Dmax, int64_t W,
                                     hipStream_t stream) {
  TTA_CHECK_ARG(n_msg >= 0 && N >= 0 && Dmax >= 0 && W > 0 && Dmax < (1 << 20) &&
                    W < (1 << 24) && n_msg < ((int64_t)1 << 31),
                "tta_segment_sum_table: sizes out of range");
  TTA_CHECK_ARG(N * W < ((int64_t)1 << 40), "tta_segment_sum_table: tensor too large");
  if (N == 0) return tta::kOk;
  TTA_CHECK_ARG(out && (Dmax == 0 || gather) && (n_msg == 0 || msg),
                "tta_segment_sum_table: null pointer");
  hipLaunchKernelGGL(k_segment_sum_table, dim3(tta_blocks(N * W, 256)), dim3(256), 0, stream, msg,
                     gather, out, N, (int)Dmax, (int)W, n_msg);
  TTA_CHECK_LAUNCH("tta_segment_sum_table");
  return tta::kOk;
}
