// Shared pieces of the MFMA GEMM kernels: argument block, epilogue codes and the epilogue that
// writes one wave's 16x16 accumulator tiles.
#pragma once

#include "common.h"
#include "../../include/tt_atom_hip_types.h"

typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

namespace tta_gemm {

enum { EPI_STORE = 0, EPI_SILU = 1, EPI_ACCUM = 2, EPI_PRE_SILU = 3, EPI_SILU_GRAD = 4,
       EPI_SIGMOID = 5, EPI_GATE = 6, EPI_GATE_BWD = 7 };

// The gate epilogue (EPI_GATE, split kernel only) of one launch: a product's output column col
// is channel h = col % H of SH coefficient c = c0 + col / H (c0 per product, GemmGroup::gc0).
// Coefficient 0 gets SiLU and its pre-activation is also stored (x0 rows, stride ldx0, H wide);
// coefficient c > 0 is multiplied by sig[row * ldg + t * H + h], the sigmoid of the gating
// columns (an earlier launch with the EPI_SIGMOID epilogue), with degree index
// t = (tab >> 4 (c - 1)) & 15 -- the GateActivation of an SO(2) convolution's output applied as
// the convolution writes it (activation.py:53-70).  EPI_GATE_BWD, the adjoint of the gate's
// input applied as the adjoint products write it (forces.py:104-130): coefficient 0 is multiplied
// by silu'(x0), coefficient c > 0 by the same sigmoid.
struct GateEpi {
  const float* sig;
  float* x0;
  int64_t ldg, ldx0;
  int H;
  unsigned tab;
};

__device__ __forceinline__ int gate_coef(const GateEpi& ge, int c0, int col) {
  return c0 + col / ge.H;
}
// gating column of coefficient c > 0, channel h
__device__ __forceinline__ int gate_gcol(const GateEpi& ge, int c, int h) {
  return (int)((ge.tab >> (4 * (c - 1))) & 15u) * ge.H + h;
}

struct GemmArgs {
  const float* A;
  const void* B;  // fp32 [K, N] (fp32 kernel) or packed fp16 / bf16 planes (split kernel)
  float* C;
  const float* bias;
  float* C2;
  const float* aux;
  int M, N, K;
  int64_t lda, ldb, ldc;
  int64_t sA, sB, sC, sBias;
  int epi;
  const float* P;  // optional row-gather table (batch 1 only)
  const int* idx0;
  const int* idx1;
  int64_t ldp, off1;
};

// Up to kMaxGroup independent products in one launch: blockIdx.z selects the product (the
// kernels of a plain call see a group of one; the fp32 kernel's strided batch uses blockIdx.z
// itself and is not combined with a group).  vec / NT32 are per product: the fp32 kernel's float4
// path and the split kernel's packed-B column tiles.
constexpr int kMaxGroup = 8;
struct GemmGroup {
  GemmArgs p[kMaxGroup];
  int NT32[kMaxGroup];
  int vec[kMaxGroup];
  int cap;  // split kernel: most blocks per product (persistent tile loop), a multiple of 8
  // split-K fp32 kernel: blockIdx.y takes k range [y * kch[z], (y + 1) * kch[z]) of product z
  // and writes its raw partial [M, N] to work + woff[z] + y * M * N
  float* work;
  int64_t woff[kMaxGroup];
  int kch[kMaxGroup];
  // EPI_GATE products: the launch's gate operands and each product's first coefficient
  GateEpi gate;
  int gc0[kMaxGroup];
};

// Accumulator layout of v_mfma_f32_16x16x{4f32,32bf16}: lane l holds D[4*(l/16)+r][l%16] in
// element r.  The epilogue is a (wave-uniform) runtime switch: one kernel symbol per tile shape.
template <int TI, int TJ>
__device__ __forceinline__ void store_tiles(const GemmArgs& p, const floatx4 (&acc)[TI][TJ],
                                            int m0, int n0, int li, int lk, float* C, float* C2,
                                            const float* aux, const float* bias) {
  const int EPI = p.epi;
#pragma unroll
  for (int j = 0; j < TJ; ++j) {
    const int col = n0 + j * 16 + li;
    if (col >= p.N) continue;
    const float bv = bias ? bias[col] : 0.f;
#pragma unroll
    for (int i = 0; i < TI; ++i) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = m0 + i * 16 + lk * 4 + r;
        if (row >= p.M) continue;
        float v = acc[i][j][r] + bv;
        if (p.P)
          v += p.P[(int64_t)p.idx0[row] * p.ldp + col] +
               p.P[(int64_t)p.idx1[row] * p.ldp + p.off1 + col];
        const int64_t off = (int64_t)row * p.ldc + col;
        if (EPI == EPI_SILU) v = tta_silu(v);
        if (EPI == EPI_SIGMOID) v = tta_sigmoid_acc(v);
        if (EPI == EPI_ACCUM) v += C[off];
        if (EPI == EPI_PRE_SILU) C2[off] = tta_silu(v);
        if (EPI == EPI_SILU_GRAD) v = v * tta_silu_grad(aux[off]);
        C[off] = v;
      }
    }
  }
}

// Accumulator layout of v_mfma_f32_32x32x16_bf16: lane l holds, in element r = 0..15,
// D[8*(r/4) + 4*(l/32) + r%4][l%32].
template <int TI, int TJ>
__device__ __forceinline__ void store_tiles32(const GemmArgs& p,
                                              const floatx16 (&acc)[TI][TJ], int m0,
                                              int n0, int l32, int lh, float* C, float* C2,
                                              const float* aux, const float* bias) {
  const int EPI = p.epi;
#pragma unroll
  for (int j = 0; j < TJ; ++j) {
    const int col = n0 + j * 32 + l32;
    if (col >= p.N) continue;
    const float bv = bias ? bias[col] : 0.f;
#pragma unroll
    for (int i = 0; i < TI; ++i) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = m0 + i * 32 + 8 * (r >> 2) + 4 * lh + (r & 3);
        if (row >= p.M) continue;
        float v = acc[i][j][r] + bv;
        if (p.P)
          v += p.P[(int64_t)p.idx0[row] * p.ldp + col] +
               p.P[(int64_t)p.idx1[row] * p.ldp + p.off1 + col];
        const int64_t off = (int64_t)row * p.ldc + col;
        if (EPI == EPI_SILU) v = tta_silu(v);
        if (EPI == EPI_SIGMOID) v = tta_sigmoid_acc(v);
        if (EPI == EPI_ACCUM) v += C[off];
        if (EPI == EPI_PRE_SILU) C2[off] = tta_silu(v);
        if (EPI == EPI_SILU_GRAD) v = v * tta_silu_grad(aux[off]);
        C[off] = v;
      }
    }
  }
}

// Split-K reduction (both GEMM kernels): C = epi(sum of the product's k-chunk partials, in chunk
// order, + bias), the epilogue of store_tiles on the partials in g.work (chunk s of product z at
// woff[z] + s * M * N, chunks of g.kch[z] k).  blockIdx.z selects the product, threads stride
// over its M x N outputs.  No row-gather term.  Internal linkage: each GEMM source has its own.
static __global__ __launch_bounds__(256) void k_splitk_reduce(GemmGroup g) {
  const GemmArgs& p = g.p[blockIdx.z];
  const int64_t MN = (int64_t)p.M * p.N;
  const int ns = (p.K + g.kch[blockIdx.z] - 1) / g.kch[blockIdx.z];
  const float* W = g.work + g.woff[blockIdx.z];
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < MN;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int row = (int)(i / p.N), col = (int)(i - (int64_t)row * p.N);
    float v = ns > 0 ? W[i] : 0.f;  // K = 0: the epilogue of a zero product
    for (int s = 1; s < ns; ++s) v += W[s * MN + i];
    if (p.bias) v += p.bias[col];
    const int64_t off = (int64_t)row * p.ldc + col;
    if (p.epi == EPI_GATE || p.epi == EPI_GATE_BWD) {
      const GateEpi& ge = g.gate;
      const int c = gate_coef(ge, g.gc0[blockIdx.z], col), h = col - (c - g.gc0[blockIdx.z]) * ge.H;
      if (c > 0) {
        v *= ge.sig[(int64_t)row * ge.ldg + gate_gcol(ge, c, h)];
      } else if (p.epi == EPI_GATE) {
        ge.x0[(int64_t)row * ge.ldx0 + h] = v;
        v = tta_silu(v);
      } else {
        v *= tta_silu_grad(ge.x0[(int64_t)row * ge.ldx0 + h]);
      }
    }
    if (p.epi == EPI_SILU) v = tta_silu(v);
    if (p.epi == EPI_SIGMOID) v = tta_sigmoid_acc(v);
    if (p.epi == EPI_ACCUM) v += p.C[off];
    if (p.epi == EPI_PRE_SILU) p.C2[off] = tta_silu(v);
    if (p.epi == EPI_SILU_GRAD) v = v * tta_silu_grad(p.aux[off]);
    p.C[off] = v;
  }
}

// XCD-aware tile order: workgroups are dispatched round-robin over the 8 XCDs, so workgroup b
// runs on XCD b % 8.  Each XCD gets a contiguous run of row-major tiles, so the column tiles of a
// row panel share that XCD's L2 and the A panel is fetched once per XCD.
__device__ __forceinline__ int xcd_tile(int ntiles) {
  const int per_xcd = (ntiles + 7) / 8;
  return (blockIdx.x % 8) * per_xcd + blockIdx.x / 8;
}

}  // namespace tta_gemm
