// fp32 GEMM on the CDNA4 matrix cores (v_mfma_f32_16x16x4_f32), for the SO(2) m-block
// contractions, the radial / edge-degree MLPs and the node-level linears of the eSCN-MD path.
//
//   C[b] = epi(A[b] (M x K, row-major, lda) * B[b] (K x N, row-major, ldb) + bias[b][N])
//
// Epilogues: 0 store; 1 store silu(v); 2 accumulate C += v; 3 store v to C and silu(v) to C2
// (pre-activation kept for the backward); 4 store v * silu'(aux) (aux shares C's layout).
// Optional row-gather term (tta_gemm_f32_gather): before the epilogue,
//   v += P[idx0[row], col] + P[idx1[row], off1 + col]        (P rows of stride ldp)
// which adds per-row node-level partial products to an edge-level GEMM.
//
// Block tiles 128x128, 64x128 or 32x64 (x16 in k), 256 threads = 4 waves in a 2x2 arrangement;
// the largest tile whose grid still fills the chip is used (dispatch()).
//
// MFMA 16x16x4 f32 operand layout (one block): lane l supplies A[l%16][l/16] and B[l/16][l%16];
// the result D[4*(l/16)+r][l%16], r=0..3, lands in accumulator element r of lane l.
#include "gemm_common.h"

#include <algorithm>

namespace {

using namespace tta_gemm;

constexpr int PAD = 4;

// Block tile BM x BN x BK with 4 waves in a WGM x WGN grid; each wave owns (BM/WGM) x (BN/WGN)
// = TI x TJ MFMA tiles of 16 x 16.  Loads stage A k-major (the 16 lanes sharing a k read 16
// consecutive rows) and B row-major in LDS; per-thread register prefetch of the next k-slab and
// two LDS buffers give one barrier per k-step.
template <int BM, int BN, int WGM, int WGN, int BK_>
struct Tile {
  static constexpr int BK = BK_;
  static constexpr int TI = BM / WGM / 16;
  static constexpr int TJ = BN / WGN / 16;
  static constexpr int A_VEC = BM * BK / 4;   // float4 loads of the A slab
  static constexpr int B_VEC = BK * BN / 4;
  static constexpr int A_PER_T = (A_VEC + 255) / 256;
  static constexpr int B_PER_T = (B_VEC + 255) / 256;
  static_assert(WGM * WGN == 4, "4 waves per block");
  static_assert(TI >= 1 && TJ >= 1, "wave tile at least 16 x 16");
};

template <class TL, int BM, bool VEC>
__device__ __forceinline__ void load_a(const GemmArgs& p, const float* A, int m0, int k0, int kmax,
                                       int t, float (&ra)[TL::A_PER_T * 4]) {
#pragma unroll
  for (int h = 0; h < TL::A_PER_T; ++h) {
    const int i = t + 256 * h;
    const int row = m0 + i / (TL::BK / 4);
    const int k = k0 + (i % (TL::BK / 4)) * 4;
    const bool in = i < TL::A_VEC && row < p.M;
    if (VEC) {
      floatx4 v = {0.f, 0.f, 0.f, 0.f};
      if (in && k < kmax) v = *reinterpret_cast<const floatx4*>(A + (int64_t)row * p.lda + k);
#pragma unroll
      for (int c = 0; c < 4; ++c) ra[4 * h + c] = v[c];
    } else {
#pragma unroll
      for (int c = 0; c < 4; ++c)
        ra[4 * h + c] = (in && k + c < kmax) ? A[(int64_t)row * p.lda + k + c] : 0.f;
    }
  }
}

template <class TL, int BN, bool VEC>
__device__ __forceinline__ void load_b(const GemmArgs& p, const float* B, int n0, int k0, int kmax,
                                       int t, float (&rb)[TL::B_PER_T * 4]) {
#pragma unroll
  for (int h = 0; h < TL::B_PER_T; ++h) {
    const int i = t + 256 * h;
    const int k = k0 + i / (BN / 4);
    const int col = n0 + (i % (BN / 4)) * 4;
    const bool in = i < TL::B_VEC && k < kmax;
    if (VEC) {
      floatx4 v = {0.f, 0.f, 0.f, 0.f};
      if (in && col < p.N) v = *reinterpret_cast<const floatx4*>(B + (int64_t)k * p.ldb + col);
#pragma unroll
      for (int c = 0; c < 4; ++c) rb[4 * h + c] = v[c];
    } else {
#pragma unroll
      for (int c = 0; c < 4; ++c)
        rb[4 * h + c] = (in && col + c < p.N) ? B[(int64_t)k * p.ldb + col + c] : 0.f;
    }
  }
}

template <class TL, int BM>
__device__ __forceinline__ void store_a(float (*As)[BM + PAD], int t,
                                        const float (&ra)[TL::A_PER_T * 4]) {
#pragma unroll
  for (int h = 0; h < TL::A_PER_T; ++h) {
    const int i = t + 256 * h;
    if (i >= TL::A_VEC) continue;
    const int r = i / (TL::BK / 4);
    const int kq = (i % (TL::BK / 4)) * 4;
#pragma unroll
    for (int c = 0; c < 4; ++c) As[kq + c][r] = ra[4 * h + c];
  }
}

template <class TL, int BN>
__device__ __forceinline__ void store_b(float (*Bs)[BN + PAD], int t,
                                        const float (&rb)[TL::B_PER_T * 4]) {
#pragma unroll
  for (int h = 0; h < TL::B_PER_T; ++h) {
    const int i = t + 256 * h;
    if (i >= TL::B_VEC) continue;
    const int kr = i / (BN / 4);
    const int nq = (i % (BN / 4)) * 4;
#pragma unroll
    for (int c = 0; c < 4; ++c) Bs[kr][nq + c] = rb[4 * h + c];
  }
}

// The epilogue is a (wave-uniform) runtime switch so every GEMM of the step is one kernel
// symbol per tile shape; it runs once per output element and costs nothing next to the K loop.
// GROUP: blockIdx.z selects the product of g (batch 1 each); otherwise g.p[0] is one strided
// batch and blockIdx.z its batch index.  SPLIT (with GROUP): blockIdx.y selects a k chunk of
// g.kch[z]; the block stores its raw partial sums for k_splitk_reduce instead of the epilogue.
template <int BM, int BN, int WGM, int WGN, int BK, bool VEC, bool GROUP, bool SPLIT = false>
__global__ __launch_bounds__(256, 2) void gemm_f32_kernel(GemmGroup g) {
  const GemmArgs& p = g.p[GROUP ? blockIdx.z : 0];
  const int64_t bz = GROUP ? 0 : blockIdx.z;
  typedef Tile<BM, BN, WGM, WGN, BK> TL;
  constexpr int TI = TL::TI, TJ = TL::TJ;
  __shared__ float As[2][BK][BM + PAD];
  __shared__ float Bs[2][BK][BN + PAD];

  const int t = threadIdx.x;
  const int lane = t & 63;
  const int wave = t >> 6;
  const int wm = wave / WGN, wn = wave % WGN;
  const int tn = (p.N + BN - 1) / BN;
  const int ntiles = tn * ((p.M + BM - 1) / BM);
  // a product of a group uses the first (ntiles rounded up to 8) blocks of the grid, so that
  // xcd_tile maps them one to one onto its tiles; wider grids belong to other products
  if ((int)blockIdx.x >= ((ntiles + 7) / 8) * 8) return;
  const int tile = xcd_tile(ntiles);
  if (tile >= ntiles) return;
  const int n0 = (tile % tn) * BN;
  const int m0 = (tile / tn) * BM;
  const float* A = p.A + bz * p.sA;
  const float* B = static_cast<const float*>(p.B) + bz * p.sB;
  float* C = p.C + bz * p.sC;
  float* C2 = p.C2 ? p.C2 + bz * p.sC : nullptr;
  const float* aux = p.aux ? p.aux + bz * p.sC : nullptr;
  const float* bias = p.bias ? p.bias + bz * p.sBias : nullptr;

  // k range of this block: the whole of K, or chunk blockIdx.y of the product's chunk length
  const int kc = SPLIT ? g.kch[blockIdx.z] : 0;
  const int kbeg = SPLIT ? (int)blockIdx.y * kc : 0;
  if (SPLIT && kbeg >= p.K) return;  // a product with fewer chunks than the grid's
  const int kend = SPLIT ? min(p.K, kbeg + kc) : p.K;

  floatx4 acc[TI][TJ];
#pragma unroll
  for (int i = 0; i < TI; ++i)
#pragma unroll
    for (int j = 0; j < TJ; ++j) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};

  float ra[TL::A_PER_T * 4], rb[TL::B_PER_T * 4];
  const int nk = (kend - kbeg + BK - 1) / BK;
  load_a<TL, BM, VEC>(p, A, m0, kbeg, kend, t, ra);
  load_b<TL, BN, VEC>(p, B, n0, kbeg, kend, t, rb);
  store_a<TL, BM>(As[0], t, ra);
  store_b<TL, BN>(Bs[0], t, rb);
  __syncthreads();

  const int li = lane & 15;
  const int lk = lane >> 4;
  const int rbase = wm * (BM / WGM), cbase = wn * (BN / WGN);
  for (int kt = 0; kt < nk; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < nk) {
      load_a<TL, BM, VEC>(p, A, m0, kbeg + (kt + 1) * BK, kend, t, ra);
      load_b<TL, BN, VEC>(p, B, n0, kbeg + (kt + 1) * BK, kend, t, rb);
    }
#pragma unroll
    for (int kk = 0; kk < BK / 4; ++kk) {
      const int k = 4 * kk + lk;
      float a[TI], b[TJ];
#pragma unroll
      for (int i = 0; i < TI; ++i) a[i] = As[buf][k][rbase + i * 16 + li];
#pragma unroll
      for (int j = 0; j < TJ; ++j) b[j] = Bs[buf][k][cbase + j * 16 + li];
#pragma unroll
      for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int j = 0; j < TJ; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[i], b[j], acc[i][j], 0, 0, 0);
    }
    if (kt + 1 < nk) {
      store_a<TL, BM>(As[buf ^ 1], t, ra);
      store_b<TL, BN>(Bs[buf ^ 1], t, rb);
    }
    __syncthreads();
  }

  if constexpr (SPLIT) {
    // raw partial of this chunk, [M, N] row-major
    float* W = g.work + g.woff[blockIdx.z] + (int64_t)blockIdx.y * p.M * p.N;
#pragma unroll
    for (int j = 0; j < TJ; ++j) {
      const int col = n0 + cbase + j * 16 + li;
      if (col >= p.N) continue;
#pragma unroll
      for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int row = m0 + rbase + i * 16 + lk * 4 + r;
          if (row < p.M) W[(int64_t)row * p.N + col] = acc[i][j][r];
        }
    }
  } else {
    store_tiles<TI, TJ>(p, acc, m0 + rbase, n0 + cbase, li, lk, C, C2, aux, bias);
  }
}

// n products (group) or one product with `batch` strided copies (n == 1, group false).
template <int BM, int BN, int WGM, int WGN, int BK>
int launch(const GemmGroup& g, int n, bool group, int64_t batch, bool vec, hipStream_t s) {
  int64_t gx = 0;
  for (int i = 0; i < n; ++i) {
    const int64_t ntiles = (int64_t)tta_blocks(g.p[i].N, BN) * tta_blocks(g.p[i].M, BM);
    if (ntiles > (1ll << 30)) {
      tta::set_error("tta_gemm_f32: grid too large");
      return tta::kBadArgument;
    }
    // one workgroup per tile, rounded up to a multiple of 8 so every XCD gets a full share
    gx = std::max(gx, ((ntiles + 7) / 8) * 8);
  }
  const dim3 grid((unsigned)gx, 1, (unsigned)(group ? n : batch));
  if (group) {
    if (vec)
      hipLaunchKernelGGL((gemm_f32_kernel<BM, BN, WGM, WGN, BK, true, true>), grid, dim3(256), 0, s,
                         g);
    else
      hipLaunchKernelGGL((gemm_f32_kernel<BM, BN, WGM, WGN, BK, false, true>), grid, dim3(256), 0, s,
                         g);
  } else {
    if (vec)
      hipLaunchKernelGGL((gemm_f32_kernel<BM, BN, WGM, WGN, BK, true, false>), grid, dim3(256), 0, s,
                         g);
    else
      hipLaunchKernelGGL((gemm_f32_kernel<BM, BN, WGM, WGN, BK, false, false>), grid, dim3(256), 0,
                         s, g);
  }
  TTA_CHECK_LAUNCH("tta_gemm_f32");
  return tta::kOk;
}

// Tile shape per call: 128 x 128 when the grid already fills the chip (>= 960 blocks, about four
// resident blocks per CU), 64 x 128 for mid-size grids, 32 x 64 for the small node-level GEMMs
// (counted over every product of a group).  The small tiles take 64-deep k steps: a grid that
// small is bound by the latency of its sequence of k steps (each waits out one round of loads),
// so a quarter of the steps, each with four times the matrix work, finishes sooner.
int dispatch(const GemmGroup& g, int n, bool group, int64_t batch, bool vec, hipStream_t s) {
  int64_t big = 0, mid = 0;
  for (int i = 0; i < n; ++i) {
    big += (int64_t)tta_blocks(g.p[i].M, 128) * tta_blocks(g.p[i].N, 128) * batch;
    mid += (int64_t)tta_blocks(g.p[i].M, 64) * tta_blocks(g.p[i].N, 128) * batch;
  }
  if (big >= 960) return launch<128, 128, 2, 2, 16>(g, n, group, batch, vec, s);
  if (mid >= 512) return launch<64, 128, 2, 2, 16>(g, n, group, batch, vec, s);
  return launch<32, 64, 2, 2, 64>(g, n, group, batch, vec, s);
}

}  // namespace

namespace {

// Checks one product and completes p (sizes); *vec: whether its float4 path applies.
int check(GemmArgs& p, int64_t M, int64_t N, int64_t K, int64_t batch, const char* name,
          bool* skip, bool* vec) {
  *skip = false;
  TTA_CHECK_ARG(M >= 0 && N >= 0 && K >= 0 && batch >= 0, "%s: negative size", name);
  TTA_CHECK_ARG(M < (int64_t)1 << 31 && N < (int64_t)1 << 31 && K < (int64_t)1 << 31,
                "%s: size exceeds int32", name);
  TTA_CHECK_ARG(tta_blocks(M, 32) <= 65535 && batch <= 65535, "%s: grid too large", name);
  TTA_CHECK_ARG(p.epi >= 0 && p.epi <= EPI_SIGMOID, "%s: bad epilogue %d", name, p.epi);
  TTA_CHECK_ARG(p.epi != EPI_PRE_SILU || p.C2, "%s: epilogue 3 needs C2", name);
  TTA_CHECK_ARG(p.epi != EPI_SILU_GRAD || p.aux, "%s: epilogue 4 needs aux", name);
  if (M == 0 || N == 0 || batch == 0) {
    *skip = true;
    return tta::kOk;
  }
  TTA_CHECK_ARG(p.A && p.B && p.C, "%s: null pointer", name);
  TTA_CHECK_ARG(p.lda >= K && p.ldb >= N && p.ldc >= N, "%s: leading dimension too small", name);
  p.M = (int)M;
  p.N = (int)N;
  p.K = (int)K;
  *vec = (K % 4 == 0) && (N % 4 == 0) && (p.lda % 4 == 0) && (p.ldb % 4 == 0) &&
         (p.sA % 4 == 0) && (p.sB % 4 == 0) && ((uintptr_t)p.A % 16 == 0) &&
         ((uintptr_t)p.B % 16 == 0);
  return tta::kOk;
}

int check_and_run(GemmArgs& p, int64_t M, int64_t N, int64_t K, int64_t batch,
                  hipStream_t stream, const char* name) {
  bool skip = false, vec = false;
  const int rc = check(p, M, N, K, batch, name, &skip, &vec);
  if (rc != tta::kOk || skip) return rc;
  GemmGroup g{};
  g.p[0] = p;
  return dispatch(g, 1, false, batch, vec, stream);
}

}  // namespace

extern "C" int tta_gemm_f32(const float* A, const float* B, float* C, const float* bias,
                            float* C2, const float* aux, int64_t M, int64_t N, int64_t K,
                            int64_t lda, int64_t ldb, int64_t ldc, int64_t batch, int64_t sA,
                            int64_t sB, int64_t sC, int64_t sBias, int epilogue,
                            hipStream_t stream) {
  GemmArgs p{A, B, C, bias, C2, aux, 0, 0, 0, lda, ldb, ldc, sA, sB, sC, sBias, epilogue,
             nullptr, nullptr, nullptr, 0, 0};
  return check_and_run(p, M, N, K, batch, stream, "tta_gemm_f32");
}

extern "C" int tta_gemm_f32_gather(const float* A, const float* B, float* C, const float* bias,
                                   float* C2, const float* aux, int64_t M, int64_t N, int64_t K,
                                   int64_t lda, int64_t ldb, int64_t ldc, const float* P,
                                   int64_t ldp, const int* idx0, const int* idx1, int64_t off1,
                                   int64_t n_rows_p, int epilogue, hipStream_t stream) {
  TTA_CHECK_ARG(P && idx0 && idx1, "tta_gemm_f32_gather: null gather pointer");
  TTA_CHECK_ARG(n_rows_p > 0 && ldp >= off1 + N && off1 >= 0,
                "tta_gemm_f32_gather: gather table too narrow");
  GemmArgs p{A, B, C, bias, C2, aux, 0, 0, 0, lda, ldb, ldc, 0, 0, 0, 0, epilogue,
             P, idx0, idx1, ldp, off1};
  return check_and_run(p, M, N, K, 1, stream, "tta_gemm_f32_gather");
}

extern "C" int tta_gemm_f32_group(const tta_gemm_problem* probs, int64_t n, hipStream_t stream) {
  TTA_CHECK_ARG(n >= 0 && n <= kMaxGroup && (probs || n == 0),
                "tta_gemm_f32_group: 0..%d products", kMaxGroup);
  GemmGroup g{};
  int m = 0;
  bool vec_all = true;
  for (int64_t i = 0; i < n; ++i) {
    const tta_gemm_problem& q = probs[i];
    TTA_CHECK_ARG(q.epilogue >= 0 && q.epilogue <= EPI_SIGMOID, "tta_gemm_f32_group: bad epilogue");
    GemmArgs p{q.A, q.B, q.C, q.bias, q.C2, q.aux, 0, 0, 0, q.lda, q.ldb, q.ldc, 0, 0, 0, 0,
               (int)q.epilogue, nullptr, nullptr, nullptr, 0, 0};
    bool skip = false, vec = false;
    const int rc = check(p, q.M, q.N, q.K, 1, "tta_gemm_f32_group", &skip, &vec);
    if (rc != tta::kOk) return rc;
    if (skip) continue;
    g.p[m++] = p;
    vec_all = vec_all && vec;
  }
  if (m == 0) return tta::kOk;
  return dispatch(g, m, true, 1, vec_all, stream);
}

// Split-K form of tta_gemm_f32_group.  A launch whose products have fewer than 160 tiles of
// 32 x 64 in all leaves most compute units idle and is bound by the latency of each
// workgroup's k loop (about 20 us at K = 1024); its products with K >= 256 then have their K cut
// into chunks (multiples of 64, at least 128) aiming at about 640 workgroups, and the others run
// as one chunk.  With more tiles the fp32 matrix rate of the launch bounds it and splitting one
// small product of a group measured slower, so nothing is split.  The decision belongs to the
// launch: a product's k sums may be ordered differently grouped and alone, while a one-chunk
// product gives the bits of tta_gemm_f32 (its partial is the whole k loop, in the same k order).
namespace {

int64_t splitk_tiles(const tta_gemm_problem* probs, int64_t n) {
  int64_t tiles = 0;
  for (int64_t i = 0; i < n; ++i)
    if (probs[i].M > 0 && probs[i].N > 0)
      tiles += tta_blocks(probs[i].M, 32) * tta_blocks(probs[i].N, 64);
  return tiles;
}

// chunk length for a product of the launch (K itself: one chunk)
int64_t splitk_chunk(int64_t K, int64_t tiles) {
  const int64_t one = std::max<int64_t>(1, K);
  if (K < 256 || tiles >= 160) return one;
  const int64_t chunks = std::min<int64_t>((640 + tiles - 1) / tiles, K / 128);
  if (chunks < 2) return one;
  return ((K + chunks - 1) / chunks + 63) / 64 * 64;
}

}  // namespace

// Workspace of tta_gemm_f32_group_splitk for these products, in floats: the sum over products
// of ceil(K / chunk) * M * N when some product takes more than one chunk, else 0 (nothing to
// gain over tta_gemm_f32_group).
extern "C" int64_t tta_gemm_f32_splitk_work(const tta_gemm_problem* probs, int64_t n) {
  if (n < 0 || n > kMaxGroup || (!probs && n > 0)) return -1;
  const int64_t tiles = splitk_tiles(probs, n);
  int64_t need = 0;
  bool split = false;
  for (int64_t i = 0; i < n; ++i) {
    const tta_gemm_problem& q = probs[i];
    if (q.M <= 0 || q.N <= 0 || q.K < 0) continue;
    const int64_t kc = splitk_chunk(q.K, tiles);
    const int64_t chunks = (q.K + kc - 1) / kc;
    split = split || chunks > 1;
    need += chunks * q.M * q.N;
  }
  return split ? need : 0;
}

extern "C" int tta_gemm_f32_group_splitk(const tta_gemm_problem* probs, int64_t n, float* work,
                                         int64_t work_floats, hipStream_t stream) {
  TTA_CHECK_ARG(n >= 0 && n <= kMaxGroup && (probs || n == 0),
                "tta_gemm_f32_group_splitk: 0..%d products", kMaxGroup);
  GemmGroup g{};
  int m = 0;
  bool vec_all = true;
  int64_t need = 0, max_chunks = 0, max_tiles = 0, max_mn = 0;
  const int64_t tiles = splitk_tiles(probs, n);
  for (int64_t i = 0; i < n; ++i) {
    const tta_gemm_problem& q = probs[i];
    TTA_CHECK_ARG(q.epilogue >= 0 && q.epilogue <= EPI_SIGMOID,
                  "tta_gemm_f32_group_splitk: bad epilogue");
    GemmArgs p{q.A, q.B, q.C, q.bias, q.C2, q.aux, 0, 0, 0, q.lda, q.ldb, q.ldc, 0, 0, 0, 0,
               (int)q.epilogue, nullptr, nullptr, nullptr, 0, 0};
    bool skip = false, vec = false;
    const int rc = check(p, q.M, q.N, q.K, 1, "tta_gemm_f32_group_splitk", &skip, &vec);
    if (rc != tta::kOk) return rc;
    if (skip) continue;
    const int64_t kc = splitk_chunk(q.K, tiles);
    const int64_t chunks = (q.K + kc - 1) / kc;
    g.kch[m] = (int)kc;
    g.woff[m] = need;
    need += chunks * q.M * q.N;
    max_chunks = std::max(max_chunks, chunks);
    max_tiles = std::max(max_tiles, (int64_t)tta_blocks(q.N, 64) * tta_blocks(q.M, 32));
    max_mn = std::max(max_mn, q.M * q.N);
    g.p[m++] = p;
    vec_all = vec_all && vec;
  }
  if (m == 0) return tta::kOk;
  TTA_CHECK_ARG(work && work_floats >= need,
                "tta_gemm_f32_group_splitk: work holds %lld floats, needs %lld",
                (long long)work_floats, (long long)need);
  TTA_CHECK_ARG(max_chunks <= 65535 && max_tiles <= (1ll << 30),
                "tta_gemm_f32_group_splitk: grid too large");
  g.work = work;
  if (max_chunks > 0) {
    const dim3 grid((unsigned)(((max_tiles + 7) / 8) * 8), (unsigned)max_chunks, (unsigned)m);
    if (vec_all)
      hipLaunchKernelGGL((gemm_f32_kernel<32, 64, 2, 2, 64, true, true, true>), grid, dim3(256), 0,
                         stream, g);
    else
      hipLaunchKernelGGL((gemm_f32_kernel<32, 64, 2, 2, 64, false, true, true>), grid, dim3(256),
                         0, stream, g);
  }
  const int64_t rb = std::min<int64_t>((max_mn + 255) / 256, 2048);
  hipLaunchKernelGGL(k_splitk_reduce, dim3((unsigned)rb, 1, (unsigned)m), dim3(256), 0, stream, g);
  TTA_CHECK_LAUNCH("tta_gemm_f32_group_splitk");
  return tta::kOk;
}
