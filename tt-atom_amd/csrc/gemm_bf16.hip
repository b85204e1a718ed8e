// Split-bf16 GEMM on the CDNA4 bf16 matrix cores (v_mfma_f32_16x16x32_bf16), fp32 accumulation.
//
//   C = epi(A (M x K fp32, row stride lda) * B (K x N, packed bf16 planes) + bias [+ row gathers])
//
// A fp32 value a is split into bf16 planes by round-to-nearest residuals:
//   a0 = bf16(a), a1 = bf16(a - a0), a2 = bf16(a - a0 - a1)        (|a - a0 - a1 - a2| <~ 2^-24 |a|)
// and B (a constant weight) was split the same way once, by tta_pack_b.  Modes:
//   mode 1: one plane each, a0 b0                        -- bf16 operands
//   mode 3: two planes each, a0b0 + a0b1 + a1b0          -- ~2^-16 relative per product
//   mode 6: three planes each, the six products of plane-exponent sum <= 2:
//           a0b0 + a0b1 + a1b0 + a0b2 + a2b0 + a1b1      -- the dropped terms are ~2^-24 relative,
//           so the result has fp32 GEMM accuracy (products of bf16 pairs are exact, the sums are
//           fp32) at 6/16 of the fp32-MFMA cost per useful flop.
//
// Packed B layout (tta_pack_b): bf16 [KT][planes][NT][64 lanes][8] with KT = ceil(K/32),
// NT = ceil(N/16): one 16(n) x 32(k) MFMA operand fragment is 1 KB, lane l holding
// B[kt*32 + 8*(l/16) + i][nt*16 + l%16], i = 0..7 (zero beyond K, N).  The A fragment of a lane
// uses the same k assignment: A[row0 + l%16][8*(l/16) + i].
//
// Block tile 128 x 128 x 32, 4 waves in 2 x 2, each wave 64 x 64 (4 x 4 MFMA tiles).  A is
// staged as fp32 in LDS (XOR-swizzled 16-byte chunks, conflict-free reads and writes) and split
// after the fragment read; B fragments are copied to LDS as packed.  Register prefetch of the
// next k-slab and double-buffered LDS give one barrier per k-step.
#include "gemm_common.h"

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

namespace {

using namespace tta_gemm;

template <int MODE>
struct Split;
template <>
struct Split<1> {
  static constexpr int NA = 1, NB = 1, NP = 1;
  static constexpr int pa[1] = {0};
  static constexpr int pb[1] = {0};
};
template <>
struct Split<3> {
  static constexpr int NA = 2, NB = 2, NP = 3;
  static constexpr int pa[3] = {0, 1, 0};
  static constexpr int pb[3] = {1, 0, 0};
};
template <>
struct Split<6> {
  // smallest terms first
  static constexpr int NA = 3, NB = 3, NP = 6;
  static constexpr int pa[6] = {1, 0, 2, 0, 1, 0};
  static constexpr int pb[6] = {1, 2, 0, 1, 0, 0};
};

template <int NPL>
__device__ __forceinline__ void split_planes(const float (&v)[8], bf16x8 (&out)[NPL]) {
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    float r = v[i];
#pragma unroll
    for (int q = 0; q < NPL; ++q) {
      const __bf16 h = (__bf16)r;
      out[q][i] = h;
      if (q + 1 < NPL) r = r - (float)h;
    }
  }
}

constexpr int BM = 128, BN = 128, BK = 32;
constexpr int NFRAG = BN / 16;  // B fragments per plane per k-step

// A slab in LDS: [128 rows][32 fp32] with the 16-byte chunk index XOR (row & 7).
__device__ __forceinline__ int a_off(int row, int chunk) {
  return row * BK + ((chunk ^ (row & 7)) << 2);
}

template <int MODE>
__global__ __launch_bounds__(256, 2) void gemm_bf16x_kernel(GemmArgs p, int NT) {
  typedef Split<MODE> S;
  constexpr int NB = S::NB, NA = S::NA;
  constexpr int TI = 4, TJ = 4;
  __shared__ float As[2][BM * BK];
  __shared__ uint4 Bs[2][NB * NFRAG * 64];

  const int t = threadIdx.x;
  const int lane = t & 63;
  const int wave = t >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int tn = (p.N + BN - 1) / BN;
  const int ntiles = tn * ((p.M + BM - 1) / BM);
  const int tile = xcd_tile(ntiles);
  if (tile >= ntiles) return;
  const int n0 = (tile % tn) * BN;
  const int m0 = (tile / tn) * BM;
  const int nt0 = n0 / 16;
  const uint4* Bp = static_cast<const uint4*>(p.B);

  floatx4 acc[TI][TJ];
#pragma unroll
  for (int i = 0; i < TI; ++i)
#pragma unroll
    for (int j = 0; j < TJ; ++j) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};

  // per-thread prefetch registers: 4 float4 of A, NB * 2 fragment chunks of B
  floatx4 ra[4];
  uint4 rb[NB * 2];
  auto load = [&](int kt) {
    const int k0 = kt * BK;
#pragma unroll
    for (int h = 0; h < 4; ++h) {
      const int c = t + 256 * h;
      const int row = m0 + (c >> 3), k = k0 + ((c & 7) << 2);
      ra[h] = (row < p.M && k < p.K)
                  ? *reinterpret_cast<const floatx4*>(p.A + (int64_t)row * p.lda + k)
                  : floatx4{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int h = 0; h < NB * 2; ++h) {
      const int c = t + 256 * h;             // chunk of the slab: plane, fragment, lane
      const int pl = c / (NFRAG * 64), f = (c / 64) % NFRAG, l = c % 64;
      rb[h] = (nt0 + f < NT) ? Bp[(((int64_t)kt * NB + pl) * NT + nt0 + f) * 64 + l]
                             : uint4{0u, 0u, 0u, 0u};
    }
  };
  auto store = [&](int buf) {
#pragma unroll
    for (int h = 0; h < 4; ++h) {
      const int c = t + 256 * h;
      *reinterpret_cast<floatx4*>(&As[buf][a_off(c >> 3, c & 7)]) = ra[h];
    }
#pragma unroll
    for (int h = 0; h < NB * 2; ++h) Bs[buf][t + 256 * h] = rb[h];
  };

  const int nk = (p.K + BK - 1) / BK;
  load(0);
  store(0);
  __syncthreads();

  const int li = lane & 15, lg = lane >> 4;
  const int rbase = wm * 64, cbase = wn * 64;
  for (int kt = 0; kt < nk; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < nk) load(kt + 1);
    bf16x8 b[TJ][NB];
#pragma unroll
    for (int j = 0; j < TJ; ++j)
#pragma unroll
      for (int q = 0; q < NB; ++q) {
        const uint4 u = Bs[buf][(q * NFRAG + wn * 4 + j) * 64 + lane];
        b[j][q] = __builtin_bit_cast(bf16x8, u);
      }
#pragma unroll
    for (int i = 0; i < TI; ++i) {
      const int row = rbase + i * 16 + li;
      const floatx4 x0 = *reinterpret_cast<const floatx4*>(&As[buf][a_off(row, 2 * lg)]);
      const floatx4 x1 = *reinterpret_cast<const floatx4*>(&As[buf][a_off(row, 2 * lg + 1)]);
      const float v[8] = {x0[0], x0[1], x0[2], x0[3], x1[0], x1[1], x1[2], x1[3]};
      bf16x8 a[NA];
      split_planes<NA>(v, a);
#pragma unroll
      for (int q = 0; q < S::NP; ++q)
#pragma unroll
        for (int j = 0; j < TJ; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[S::pa[q]], b[j][S::pb[q]],
                                                              acc[i][j], 0, 0, 0);
    }
    if (kt + 1 < nk) store(buf ^ 1);
    __syncthreads();
  }
  store_tiles<TI, TJ>(p, acc, m0 + rbase, n0 + cbase, li, lg, p.C, p.C2, p.aux, p.bias);
}

// Pack B [K, N] (row stride ldb) into `planes` bf16 planes in fragment order; one thread per
// (kt, nt, lane) writes the 8 values of every plane.
__global__ __launch_bounds__(256) void k_pack_b(const float* __restrict__ B, int K, int N,
                                                int64_t ldb, int planes, int KT, int NT,
                                                uint4* __restrict__ out) {
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= (int64_t)KT * NT * 64) return;
  const int l = (int)(gid % 64);
  const int nt = (int)((gid / 64) % NT);
  const int kt = (int)(gid / (64 * NT));
  const int n = nt * 16 + (l & 15);
  float r[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int k = kt * 32 + 8 * (l >> 4) + i;
    r[i] = (k < K && n < N) ? B[(int64_t)k * ldb + n] : 0.f;
  }
  for (int q = 0; q < planes; ++q) {
    bf16x8 h;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      h[i] = (__bf16)r[i];
      r[i] -= (float)h[i];
    }
    out[(((int64_t)kt * planes + q) * NT + nt) * 64 + l] = __builtin_bit_cast(uint4, h);
  }
}

template <int MODE>
int launch_bf16x(const GemmArgs& p, int NT, hipStream_t s) {
  const int64_t ntiles = (int64_t)tta_blocks(p.N, BN) * tta_blocks(p.M, BM);
  if (ntiles > (1ll << 30)) {
    tta::set_error("tta_gemm_bf16x: grid too large");
    return tta::kBadArgument;
  }
  hipLaunchKernelGGL(gemm_bf16x_kernel<MODE>, dim3((unsigned)(((ntiles + 7) / 8) * 8)), dim3(256),
                     0, s, p, NT);
  TTA_CHECK_LAUNCH("tta_gemm_bf16x");
  return tta::kOk;
}

int planes_of(int mode) { return mode == 1 ? 1 : mode == 3 ? 2 : mode == 6 ? 3 : 0; }

}  // namespace

extern "C" int64_t tta_pack_b_elems(int64_t K, int64_t N, int mode) {
  const int pl = planes_of(mode);
  if (pl == 0 || K <= 0 || N <= 0) return -1;
  return ((K + 31) / 32) * ((N + 15) / 16) * 512 * pl;
}

extern "C" int tta_pack_b(const float* B, int64_t K, int64_t N, int64_t ldb, int mode,
                          void* out, int64_t out_elems, hipStream_t stream) {
  const int pl = planes_of(mode);
  TTA_CHECK_ARG(pl > 0, "tta_pack_b: mode must be 1, 3 or 6 (got %d)", mode);
  TTA_CHECK_ARG(K > 0 && N > 0 && K < (1 << 30) && N < (1 << 30) && ldb >= N,
                "tta_pack_b: bad sizes");
  TTA_CHECK_ARG(out_elems == tta_pack_b_elems(K, N, mode), "tta_pack_b: output has %lld bf16, "
                "expected %lld", (long long)out_elems, (long long)tta_pack_b_elems(K, N, mode));
  TTA_CHECK_ARG(B && out && ((uintptr_t)out % 16 == 0), "tta_pack_b: null or misaligned pointer");
  const int KT = (int)((K + 31) / 32), NT = (int)((N + 15) / 16);
  hipLaunchKernelGGL(k_pack_b, dim3(tta_blocks((int64_t)KT * NT * 64, 256)), dim3(256), 0, stream,
                     B, (int)K, (int)N, ldb, pl, KT, NT, static_cast<uint4*>(out));
  TTA_CHECK_LAUNCH("tta_pack_b");
  return tta::kOk;
}

extern "C" int tta_gemm_bf16x(const float* A, const void* Bp, float* C, const float* bias,
                              float* C2, const float* aux, int64_t M, int64_t N, int64_t K,
                              int64_t lda, int64_t ldc, int mode, const float* P, int64_t ldp,
                              const int* idx0, const int* idx1, int64_t off1, int64_t n_rows_p,
                              int epilogue, hipStream_t stream) {
  TTA_CHECK_ARG(planes_of(mode) > 0, "tta_gemm_bf16x: mode must be 1, 3 or 6 (got %d)", mode);
  TTA_CHECK_ARG(M >= 0 && N >= 0 && K >= 0, "tta_gemm_bf16x: negative size");
  TTA_CHECK_ARG(M < (int64_t)1 << 31 && N < (int64_t)1 << 30 && K < (int64_t)1 << 30,
                "tta_gemm_bf16x: size exceeds int32");
  TTA_CHECK_ARG(epilogue >= 0 && epilogue <= 4, "tta_gemm_bf16x: bad epilogue %d", epilogue);
  TTA_CHECK_ARG(epilogue != EPI_PRE_SILU || C2, "tta_gemm_bf16x: epilogue 3 needs C2");
  TTA_CHECK_ARG(epilogue != EPI_SILU_GRAD || aux, "tta_gemm_bf16x: epilogue 4 needs aux");
  TTA_CHECK_ARG(!P || (idx0 && idx1 && n_rows_p > 0 && off1 >= 0 && ldp >= off1 + N),
                "tta_gemm_bf16x: bad row-gather table");
  if (M == 0 || N == 0) return tta::kOk;
  TTA_CHECK_ARG(A && Bp && C, "tta_gemm_bf16x: null pointer");
  TTA_CHECK_ARG(K % 4 == 0 && lda % 4 == 0 && (uintptr_t)A % 16 == 0,
                "tta_gemm_bf16x: A needs K, lda multiples of 4 and 16-byte alignment");
  TTA_CHECK_ARG(lda >= K && ldc >= N, "tta_gemm_bf16x: leading dimension too small");
  TTA_CHECK_ARG((uintptr_t)Bp % 16 == 0, "tta_gemm_bf16x: packed B must be 16-byte aligned");
  GemmArgs p{A, Bp, C, bias, C2, aux, (int)M, (int)N, (int)K, lda, 0, ldc, 0, 0, 0, 0, epilogue,
             P, idx0, idx1, ldp, off1};
  const int NT = (int)((N + 15) / 16);
  switch (mode) {
    case 1: return launch_bf16x<1>(p, NT, stream);
    case 3: return launch_bf16x<3>(p, NT, stream);
    default: return launch_bf16x<6>(p, NT, stream);
  }
}
