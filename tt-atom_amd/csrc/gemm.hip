// fp32 GEMM on the CDNA4 matrix cores (v_mfma_f32_16x16x4_f32), for the SO(2) m-block
// contractions, the radial / edge-degree MLPs and the node-level linears of the eSCN-MD path.
//
//   C[b] = epi(A[b] (M x K, row-major, lda) * B[b] (K x N, row-major, ldb) + bias[b][N])
//
// Epilogues: 0 store; 1 store silu(v); 2 accumulate C += v; 3 store v to C and silu(v) to C2
// (pre-activation kept for the backward); 4 store v * silu'(aux) (aux shares C's layout).
//
// Block tile 128x128x16, 256 threads = 4 waves in a 2x2 arrangement, each wave owns a 64x64
// sub-tile = 4x4 MFMA tiles of 16x16 (16 fp32x4 accumulators).  A is staged k-major in LDS so
// that the 16 lanes sharing a k read 16 consecutive rows; B is staged row-major.  Two LDS
// buffers with register prefetch of the next k-slab give one barrier per k-step.
//
// MFMA 16x16x4 f32 operand layout (one block): lane l supplies A[l%16][l/16] and B[l/16][l%16];
// the result D[4*(l/16)+r][l%16], r=0..3, lands in accumulator element r of lane l.
#include "common.h"

typedef float floatx4 __attribute__((ext_vector_type(4)));

namespace {

constexpr int BM = 128, BN = 128, BK = 16, PAD = 4;

struct GemmArgs {
  const float* A;
  const float* B;
  float* C;
  const float* bias;
  float* C2;
  const float* aux;
  int M, N, K;
  int64_t lda, ldb, ldc;
  int64_t sA, sB, sC, sBias;
  int epi;
};

enum { EPI_STORE = 0, EPI_SILU = 1, EPI_ACCUM = 2, EPI_PRE_SILU = 3, EPI_SILU_GRAD = 4 };

template <bool VEC>
__device__ __forceinline__ void load_a(const GemmArgs& p, const float* A, int m0, int k0, int t,
                                       float (&ra)[8]) {
  const int kq = (t & 3) * 4;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int r = (t >> 2) + 64 * h;
    const int row = m0 + r;
    const int k = k0 + kq;
    if (VEC) {
      floatx4 v = {0.f, 0.f, 0.f, 0.f};
      if (row < p.M && k < p.K) v = *reinterpret_cast<const floatx4*>(A + (int64_t)row * p.lda + k);
      ra[4 * h + 0] = v[0];
      ra[4 * h + 1] = v[1];
      ra[4 * h + 2] = v[2];
      ra[4 * h + 3] = v[3];
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        ra[4 * h + i] = (row < p.M && k + i < p.K) ? A[(int64_t)row * p.lda + k + i] : 0.f;
    }
  }
}

template <bool VEC>
__device__ __forceinline__ void load_b(const GemmArgs& p, const float* B, int n0, int k0, int t,
                                       float (&rb)[8]) {
  const int nq = (t & 31) * 4;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int kr = (t >> 5) + 8 * h;
    const int k = k0 + kr;
    const int col = n0 + nq;
    if (VEC) {
      floatx4 v = {0.f, 0.f, 0.f, 0.f};
      if (k < p.K && col < p.N) v = *reinterpret_cast<const floatx4*>(B + (int64_t)k * p.ldb + col);
      rb[4 * h + 0] = v[0];
      rb[4 * h + 1] = v[1];
      rb[4 * h + 2] = v[2];
      rb[4 * h + 3] = v[3];
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        rb[4 * h + i] = (k < p.K && col + i < p.N) ? B[(int64_t)k * p.ldb + col + i] : 0.f;
    }
  }
}

__device__ __forceinline__ void store_a(float (*As)[BM + PAD], int t, const float (&ra)[8]) {
  const int kq = (t & 3) * 4;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int r = (t >> 2) + 64 * h;
#pragma unroll
    for (int i = 0; i < 4; ++i) As[kq + i][r] = ra[4 * h + i];
  }
}

__device__ __forceinline__ void store_b(float (*Bs)[BN + PAD], int t, const float (&rb)[8]) {
  const int nq = (t & 31) * 4;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int kr = (t >> 5) + 8 * h;
#pragma unroll
    for (int i = 0; i < 4; ++i) Bs[kr][nq + i] = rb[4 * h + i];
  }
}

// The epilogue is a (wave-uniform) runtime switch so every GEMM of the step is one kernel
// symbol; it runs once per output element and costs nothing next to the K loop.
template <bool VEC>
__global__ __launch_bounds__(256, 2) void gemm_f32_kernel(GemmArgs p) {
  const int EPI = p.epi;
  __shared__ float As[2][BK][BM + PAD];
  __shared__ float Bs[2][BK][BN + PAD];

  const int t = threadIdx.x;
  const int lane = t & 63;
  const int wave = t >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int n0 = blockIdx.x * BN;
  const int m0 = blockIdx.y * BM;
  const float* A = p.A + (int64_t)blockIdx.z * p.sA;
  const float* B = p.B + (int64_t)blockIdx.z * p.sB;
  float* C = p.C + (int64_t)blockIdx.z * p.sC;
  float* C2 = p.C2 ? p.C2 + (int64_t)blockIdx.z * p.sC : nullptr;
  const float* aux = p.aux ? p.aux + (int64_t)blockIdx.z * p.sC : nullptr;
  const float* bias = p.bias ? p.bias + (int64_t)blockIdx.z * p.sBias : nullptr;

  floatx4 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};

  float ra[8], rb[8];
  const int nk = (p.K + BK - 1) / BK;
  load_a<VEC>(p, A, m0, 0, t, ra);
  load_b<VEC>(p, B, n0, 0, t, rb);
  store_a(As[0], t, ra);
  store_b(Bs[0], t, rb);
  __syncthreads();

  const int li = lane & 15;
  const int lk = lane >> 4;
  for (int kt = 0; kt < nk; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < nk) {
      load_a<VEC>(p, A, m0, (kt + 1) * BK, t, ra);
      load_b<VEC>(p, B, n0, (kt + 1) * BK, t, rb);
    }
#pragma unroll
    for (int kk = 0; kk < BK / 4; ++kk) {
      const int k = 4 * kk + lk;
      float a[4], b[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) a[i] = As[buf][k][wm * 64 + i * 16 + li];
#pragma unroll
      for (int j = 0; j < 4; ++j) b[j] = Bs[buf][k][wn * 64 + j * 16 + li];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[i], b[j], acc[i][j], 0, 0, 0);
    }
    if (kt + 1 < nk) {
      store_a(As[buf ^ 1], t, ra);
      store_b(Bs[buf ^ 1], t, rb);
    }
    __syncthreads();
  }

#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int col = n0 + wn * 64 + j * 16 + li;
    if (col >= p.N) continue;
    const float bv = bias ? bias[col] : 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = m0 + wm * 64 + i * 16 + lk * 4 + r;
        if (row >= p.M) continue;
        float v = acc[i][j][r] + bv;
        const int64_t off = (int64_t)row * p.ldc + col;
        if (EPI == EPI_SILU) v = tta_silu(v);
        if (EPI == EPI_ACCUM) v += C[off];
        if (EPI == EPI_PRE_SILU) C2[off] = tta_silu(v);
        if (EPI == EPI_SILU_GRAD) v = v * tta_silu_grad(aux[off]);
        C[off] = v;
      }
    }
  }
}

int launch(const GemmArgs& p, int64_t batch, bool vec, hipStream_t s) {
  dim3 grid(tta_blocks(p.N, BN), tta_blocks(p.M, BM), (unsigned)batch);
  if (vec)
    hipLaunchKernelGGL((gemm_f32_kernel<true>), grid, dim3(256), 0, s, p);
  else
    hipLaunchKernelGGL((gemm_f32_kernel<false>), grid, dim3(256), 0, s, p);
  TTA_CHECK_LAUNCH("tta_gemm_f32");
  return tta::kOk;
}

}  // namespace

extern "C" int tta_gemm_f32(const float* A, const float* B, float* C, const float* bias,
                            float* C2, const float* aux, int64_t M, int64_t N, int64_t K,
                            int64_t lda, int64_t ldb, int64_t ldc, int64_t batch, int64_t sA,
                            int64_t sB, int64_t sC, int64_t sBias, int epilogue,
                            hipStream_t stream) {
  TTA_CHECK_ARG(M >= 0 && N >= 0 && K >= 0 && batch >= 0, "tta_gemm_f32: negative size");
  TTA_CHECK_ARG(M < (int64_t)1 << 31 && N < (int64_t)1 << 31 && K < (int64_t)1 << 31,
                "tta_gemm_f32: size exceeds int32");
  TTA_CHECK_ARG(tta_blocks(M, BM) <= 65535 && batch <= 65535, "tta_gemm_f32: grid too large");
  TTA_CHECK_ARG(epilogue >= 0 && epilogue <= 4, "tta_gemm_f32: bad epilogue %d", epilogue);
  TTA_CHECK_ARG(epilogue != EPI_PRE_SILU || C2, "tta_gemm_f32: epilogue 3 needs C2");
  TTA_CHECK_ARG(epilogue != EPI_SILU_GRAD || aux, "tta_gemm_f32: epilogue 4 needs aux");
  if (M == 0 || N == 0 || batch == 0) return tta::kOk;
  TTA_CHECK_ARG(A && B && C, "tta_gemm_f32: null pointer");
  TTA_CHECK_ARG(lda >= K && ldb >= N && ldc >= N, "tta_gemm_f32: leading dimension too small");
  GemmArgs p{A, B, C, bias, C2, aux, (int)M, (int)N, (int)K, lda, ldb, ldc, sA, sB, sC, sBias,
             epilogue};
  const bool vec = (K % 4 == 0) && (N % 4 == 0) && (lda % 4 == 0) && (ldb % 4 == 0) &&
                   (sA % 4 == 0) && (sB % 4 == 0) && ((uintptr_t)A % 16 == 0) &&
                   ((uintptr_t)B % 16 == 0);
  return launch(p, batch, vec, stream);
}
