// Split-bf16 GEMM on the CDNA4 bf16 matrix cores (v_mfma_f32_32x32x16_bf16), fp32 accumulation.
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
// The 32x32x16 instruction: measured on MI355X it sustains about twice the bf16 rate of
// 16x16x32 (which issues at half rate).  Operand layout: lane l supplies A[l%32][8*(l/32) + e] and
// B[8*(l/32) + e][l%32], e = 0..7, of a 32 x 16 / 16 x 32 block.
//
// Packed B layout (tta_pack_b): bf16 [KT][planes][NT32][2][64 lanes][8] with KT = ceil(K/32),
// NT32 = ceil(N/32): one 16(k) x 32(n) fragment is 1 KB, lane l holding
// B[kt*32 + ks*16 + 8*(l/32) + e][n32*32 + l%32] (zero beyond K, N).
//
// Block tile (64 WM) x 128 x 32: WM x 2 waves, each 64 x 64 (2 x 2 MFMA tiles of 32 x 32).  The
// A slab is split while it is written to LDS (one bf16 plane array per plane, 16-byte chunks
// XOR-swizzled over 16 rows so that neither the fragment reads nor the writes conflict); the B
// slab is copied as packed.  Register prefetch of the next slab and double-buffered LDS give one
// barrier per k-step.  WM = 4 (256 x 128, 512 threads) for the split modes, WM = 2 for bf16.
#include "gemm_common.h"

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));

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

template <int NPL, int L>
__device__ __forceinline__ void split_planes(const float* v, __bf16 (&out)[NPL][L]) {
#pragma unroll
  for (int i = 0; i < L; ++i) {
    float r = v[i];
#pragma unroll
    for (int q = 0; q < NPL; ++q) {
      const __bf16 h = (__bf16)r;
      out[q][i] = h;
      if (q + 1 < NPL) r = r - (float)h;
    }
  }
}

constexpr int BN = 128, BK = 32;
constexpr int NF = (BN / 32) * 2;  // B fragments per plane per k-step: n32 tiles x k16 halves

// 16-byte chunk swizzle of a 64-byte bf16 row: conflict-free for any 16 consecutive rows read
// at one logical chunk (and for 8-row groups).
__device__ __forceinline__ int swz(int row) { return ((row >> 1) ^ (row >> 2)) & 3; }

__device__ __forceinline__ float epi_one(const GemmArgs& p, float v, int row, int col) {
  if (p.bias) v += p.bias[col];
  if (p.P)
    v += p.P[(int64_t)p.idx0[row] * p.ldp + col] + p.P[(int64_t)p.idx1[row] * p.ldp + p.off1 + col];
  const int64_t off = (int64_t)row * p.ldc + col;
  if (p.epi == EPI_SILU) v = tta_silu(v);
  if (p.epi == EPI_ACCUM) v += p.C[off];
  if (p.epi == EPI_PRE_SILU) p.C2[off] = tta_silu(v);
  if (p.epi == EPI_SILU_GRAD) v = v * tta_silu_grad(p.aux[off]);
  return v;
}

// Rows [row0, row0 + rows) of a 128-column output tile staged in LDS (row stride ldt floats):
// thread t takes float4 column groups t, t + nth, ...; vec_ok (host-checked 16-byte alignment of
// every operand row) selects the float4 path.
__device__ __forceinline__ void epilogue_rows(const GemmArgs& p, const float* Ct, int ldt, int rows,
                                           int row0, int n0, int t, int nth, bool vec_ok) {
#pragma unroll 1
  for (int idx = t; idx < rows * (BN / 4); idx += nth) {
    const int rr = idx / (BN / 4), c4 = idx % (BN / 4);
    const int row = row0 + rr, col = n0 + 4 * c4;
    if (row >= p.M || col >= p.N) continue;
    const floatx4 a = *reinterpret_cast<const floatx4*>(Ct + rr * ldt + 4 * c4);
    const int64_t off = (int64_t)row * p.ldc + col;
    if (vec_ok && col + 3 < p.N) {
      floatx4 v = a;
      if (p.bias) v += *reinterpret_cast<const floatx4*>(p.bias + col);
      if (p.P)
        v += *reinterpret_cast<const floatx4*>(p.P + (int64_t)p.idx0[row] * p.ldp + col) +
             *reinterpret_cast<const floatx4*>(p.P + (int64_t)p.idx1[row] * p.ldp + p.off1 + col);
      if (p.epi == EPI_ACCUM) v += *reinterpret_cast<const floatx4*>(p.C + off);
      if (p.epi == EPI_SILU || p.epi == EPI_PRE_SILU || p.epi == EPI_SILU_GRAD) {
        floatx4 w = v;
        const floatx4 x = p.epi == EPI_SILU_GRAD ? *reinterpret_cast<const floatx4*>(p.aux + off)
                                                 : v;
#pragma unroll
        for (int e = 0; e < 4; ++e)
          w[e] = p.epi == EPI_SILU_GRAD ? v[e] * tta_silu_grad(x[e]) : tta_silu(v[e]);
        if (p.epi == EPI_PRE_SILU)
          *reinterpret_cast<floatx4*>(p.C2 + off) = w;
        else
          v = w;
      }
      *reinterpret_cast<floatx4*>(p.C + off) = v;
    } else {
      for (int e = 0; e < 4 && col + e < p.N; ++e) p.C[off + e] = epi_one(p, a[e], row, col + e);
    }
  }
}

template <int WM, int MODE>
__global__ __launch_bounds__(128 * WM, WM == 2 ? 2 : 1) void gemm_bf16x_kernel(GemmArgs p,
                                                                               int NT32,
                                                                               bool vec_ok) {
  typedef Split<MODE> S;
  constexpr int NA = S::NA, NB = S::NB;
  constexpr int BM = 64 * WM, NTH = 128 * WM;
  constexpr int BPT = NB * NF * 64 / NTH;  // B slab chunks per thread
  static_assert(BPT * NTH == NB * NF * 64, "B slab must split evenly over the threads");
  constexpr int A_SLAB = NA * BM * 4, B_SLAB = NB * NF * 64;  // in 16-byte chunks
  // [A slab x 2 | B slab x 2]; plane q of an A slab: BM rows x 4 chunks of 16 B (32 bf16).
  // After the k-loop the same memory stages the output tile for the epilogue.
  __shared__ uint4 smem[2 * (A_SLAB + B_SLAB)];
  auto As = [&](int b) { return smem + b * A_SLAB; };
  auto Bs = [&](int b) { return smem + 2 * A_SLAB + b * B_SLAB; };

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
  const int nt0 = n0 / 32;
  const uint4* Bp = static_cast<const uint4*>(p.B);

  floatx16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  floatx4 ra[4];
  uint4 rb[BPT];
  auto load = [&](int kt) {
    const int k0 = kt * BK;
#pragma unroll
    for (int h = 0; h < 4; ++h) {
      const int c = t + NTH * h;
      const int row = m0 + (c >> 3), k = k0 + ((c & 7) << 2);
      ra[h] = (row < p.M && k < p.K)
                  ? *reinterpret_cast<const floatx4*>(p.A + (int64_t)row * p.lda + k)
                  : floatx4{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int h = 0; h < BPT; ++h) {
      const int c = t + NTH * h;  // slab chunk: plane, fragment (n32 * 2 + k16 half), lane
      const int pl = c / (NF * 64), f = (c / 64) % NF, l = c % 64;
      rb[h] = (nt0 + (f >> 1) < NT32)
                  ? Bp[((((int64_t)kt * NB + pl) * NT32 + nt0 + (f >> 1)) * 2 + (f & 1)) * 64 + l]
                  : uint4{0u, 0u, 0u, 0u};
    }
  };
  auto store = [&](int buf) {
#pragma unroll
    for (int h = 0; h < 4; ++h) {
      const int c = t + NTH * h;
      const int row = c >> 3, kq = c & 7;
      const float v[4] = {ra[h][0], ra[h][1], ra[h][2], ra[h][3]};
      __bf16 pl[NA][4];
      split_planes<NA, 4>(v, pl);
      const int ch = (kq >> 1) ^ swz(row);
#pragma unroll
      for (int q = 0; q < NA; ++q) {
        const bf16x4 w = {pl[q][0], pl[q][1], pl[q][2], pl[q][3]};
        *reinterpret_cast<bf16x4*>(reinterpret_cast<char*>(&As(buf)[(q * BM + row) * 4 + ch]) +
                                   (kq & 1) * 8) = w;
      }
    }
#pragma unroll
    for (int h = 0; h < BPT; ++h) Bs(buf)[t + NTH * h] = rb[h];
  };

  const int nk = (p.K + BK - 1) / BK;
  load(0);
  store(0);
  __syncthreads();

  const int l32 = lane & 31, lh = lane >> 5;
  const int rbase = wm * 64, cbase = wn * 64;
  for (int kt = 0; kt < nk; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < nk) load(kt + 1);
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      bf16x8 b[2][NB], a[2][NA];
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int q = 0; q < NB; ++q)
          b[j][q] = __builtin_bit_cast(bf16x8,
                                       Bs(buf)[(q * NF + (wn * 2 + j) * 2 + ks) * 64 + lane]);
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int row = rbase + i * 32 + l32;
        const int ch = (2 * ks + lh) ^ swz(row);
#pragma unroll
        for (int q = 0; q < NA; ++q)
          a[i][q] = __builtin_bit_cast(bf16x8, As(buf)[(q * BM + row) * 4 + ch]);
      }
#pragma unroll
      for (int q = 0; q < S::NP; ++q)
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
          for (int j = 0; j < 2; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i][S::pa[q]], b[j][S::pb[q]],
                                                                acc[i][j], 0, 0, 0);
    }
    if (kt + 1 < nk) store(buf ^ 1);
    __syncthreads();
  }
  // Epilogue: stage the accumulators through LDS in row passes, then each thread applies the
  // epilogue to whole float4 column groups and writes coalesced rows.
  constexpr int LDT = BN + 8;  // row stride (floats): lanes 32..63 (rows +4) land 32 banks away
  constexpr int SMEM_F = 2 * (A_SLAB + B_SLAB) * 4;
  constexpr int RP = (BM * LDT <= SMEM_F) ? BM : (BM / 2 * LDT <= SMEM_F) ? BM / 2
                   : (BM / 4 * LDT <= SMEM_F) ? BM / 4 : 32;
  static_assert(RP % 32 == 0 && RP * LDT <= SMEM_F, "epilogue staging must fit the LDS buffer");
  float* Ct = reinterpret_cast<float*>(smem);
  for (int r0 = 0; r0 < BM; r0 += RP) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int rt = rbase + i * 32 - r0;  // row tile start inside this pass
      if (rt < 0 || rt >= RP) continue;
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r)
          Ct[(rt + 8 * (r >> 2) + 4 * lh + (r & 3)) * LDT + cbase + j * 32 + l32] = acc[i][j][r];
    }
    __syncthreads();
    epilogue_rows(p, Ct, LDT, RP, m0 + r0, n0, t, NTH, vec_ok);
    __syncthreads();
  }
}

// Pack B [K, N] (row stride ldb) into `planes` bf16 planes in fragment order; one thread per
// (kt, n32, k16 half, lane) writes the 8 values of every plane.
__global__ __launch_bounds__(256) void k_pack_b(const float* __restrict__ B, int K, int N,
                                                int64_t ldb, int planes, int KT, int NT32,
                                                uint4* __restrict__ out) {
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= (int64_t)KT * NT32 * 128) return;
  const int l = (int)(gid % 64);
  const int ks = (int)((gid / 64) % 2);
  const int nt = (int)((gid / 128) % NT32);
  const int kt = (int)(gid / (128 * (int64_t)NT32));
  const int n = nt * 32 + (l & 31);
  float r[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int k = kt * 32 + ks * 16 + 8 * (l >> 5) + e;
    r[e] = (k < K && n < N) ? B[(int64_t)k * ldb + n] : 0.f;
  }
  for (int q = 0; q < planes; ++q) {
    bf16x8 h;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      h[e] = (__bf16)r[e];
      r[e] -= (float)h[e];
    }
    out[((((int64_t)kt * planes + q) * NT32 + nt) * 2 + ks) * 64 + l] = __builtin_bit_cast(uint4, h);
  }
}

template <int WM, int MODE>
int launch_bf16x(const GemmArgs& p, int NT32, hipStream_t s) {
  const int64_t ntiles = (int64_t)tta_blocks(p.N, BN) * tta_blocks(p.M, 64 * WM);
  if (ntiles > (1ll << 30)) {
    tta::set_error("tta_gemm_bf16x: grid too large");
    return tta::kBadArgument;
  }
  auto al = [](const void* q) { return q == nullptr || (uintptr_t)q % 16 == 0; };
  const bool vec_ok = p.N % 4 == 0 && p.ldc % 4 == 0 && al(p.C) && al(p.C2) && al(p.aux) &&
                      al(p.bias) && (!p.P || (al(p.P) && p.ldp % 4 == 0 && p.off1 % 4 == 0));
  hipLaunchKernelGGL((gemm_bf16x_kernel<WM, MODE>), dim3((unsigned)(((ntiles + 7) / 8) * 8)),
                     dim3(128 * WM), 0, s, p, NT32, vec_ok);
  TTA_CHECK_LAUNCH("tta_gemm_bf16x");
  return tta::kOk;
}

int planes_of(int mode) { return mode == 1 ? 1 : mode == 3 ? 2 : mode == 6 ? 3 : 0; }

}  // namespace

extern "C" int64_t tta_pack_b_elems(int64_t K, int64_t N, int mode) {
  const int pl = planes_of(mode);
  if (pl == 0 || K <= 0 || N <= 0) return -1;
  return ((K + 31) / 32) * ((N + 31) / 32) * 1024 * pl;
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
  const int KT = (int)((K + 31) / 32), NT32 = (int)((N + 31) / 32);
  hipLaunchKernelGGL(k_pack_b, dim3(tta_blocks((int64_t)KT * NT32 * 128, 256)), dim3(256), 0,
                     stream, B, (int)K, (int)N, ldb, pl, KT, NT32, static_cast<uint4*>(out));
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
  const int NT32 = (int)((N + 31) / 32);
  switch (mode) {
    case 1: return launch_bf16x<2, 1>(p, NT32, stream);
    case 3: return launch_bf16x<4, 3>(p, NT32, stream);
    default: return launch_bf16x<4, 6>(p, NT32, stream);
  }
}
