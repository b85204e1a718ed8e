// Fused node-level kernels of the eSCN-MD step (uma-s-1: spectral feed-forward), one launch per
// stage instead of a chain of small ones:
//
//   k_spectral_block_fwd   x2 = x1 + SpectralAtomwise(RMSNormSH_2(x1))          (model.py:158-172,
//                          norm.py:93-111, spectral.py:146-188), optionally followed by the next
//                          RMSNormSH (the next block's norm_1 with the system embedding added to
//                          coefficient 0, or the final norm): 6 launches -> 1 per block
//   k_spectral_block_bwd   the reverse: the next norm's backward plus the residual adjoint, then
//                          the spectral FF and norm_2 backward (forces.py:49-98, 258-346) plus the
//                          residual: 6 -> 1 per block
//   k_energy_head_fwd      per-node energy MLP on coefficient 0 (model.py:223-235)
//   k_energy_head_bwd      its adjoint seeded with dE/dnode_e = 1 (forces.py:438-461)
//
// A workgroup owns NT = 16 nodes.  Their rows live in LDS as [coefficient][node][channel] (row
// stride C + 4 floats: the 16 rows of an MFMA A fragment then fall in distinct banks), and every
// product is a per-coefficient matrix product on the fp32 matrix cores
// (v_mfma_f32_16x16x4_f32): rows = the 16 nodes of one coefficient, the weight of the
// coefficient's degree l as the B operand, read from global memory (the weights are shared by
// every workgroup and stay in L2).  Lane l supplies A[l%16][l/16] and B[l/16][l%16]; the result
// D[4*(l/16)+r][l%16] lands in accumulator element r.  Each wave owns whole 16-column output
// tiles for all nine coefficients, so the gate's per-degree sums over coefficients are
// register-local.  Per-node norms run one wavefront per node (64 lanes x 2 channels).
//
// Requirements (checked on the host): C and H multiples of 16, at most 128; lmax = 2.
#include "common.h"

#include <atomic>

namespace {

typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int NT = 16;        // nodes per workgroup
constexpr int NW = 8;         // waves per workgroup
constexpr int NTH = 64 * NW;
constexpr int NS = NT / NW;   // nodes per wave in the per-node phases
constexpr int CMAX = 128;     // largest C / H
constexpr int LDP = CMAX + 4; // LDS row stride (floats) of the [coef][node][channel] buffer
constexpr int MAXJ = (CMAX / 16 + NW - 1) / NW;  // output column tiles per wave

__device__ __forceinline__ int ndeg(int j) { return j == 0 ? 0 : (j < 4 ? 1 : 2); }
__device__ __forceinline__ float nbdw(int j) {
  const int l = ndeg(j);
  return (float)(1.0 / (2 * l + 1) / 3.0);
}
__device__ __forceinline__ floatx4 mfma4(float a, float b, floatx4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// LDS row of (coefficient c, local node r)
__device__ __forceinline__ float* lrow(float* buf, int c, int r) { return buf + (c * NT + r) * LDP; }

// acc[c][jj] (+)= X[c] (16 x K, LDS rows at stride ldx) @ W[deg(c)] (K x Nout, row-major at
// ldw, per-degree stride dstride) for the column tiles j = wave + NW jj of the Nout / 16 tiles;
// NC = 9 (all coefficients) or 1 (coefficient 0 only, degree 0 weight).  A wave whose j is past
// the last tile (narrow layers only) recomputes a valid tile and its caller discards the result,
// so the inner loop has no branches.  K runs in chunks of 16: in MFMA step s of a chunk, slot q
// (= lane / 16) of both operands is k = k0 + 4 q + s, so a lane reads its A values of a chunk as
// one float4 from LDS.  The B values arrive D chunks at a time, the next D chunks' loads in
// flight while the current ones are multiplied: D = 1 suffices when nine coefficients' MFMAs
// cover a load (NC = 9); the single-coefficient products take D = 4 (K a multiple of 64) so
// that their short chunks do not each wait out a load.
template <int NC, int D>
__device__ __forceinline__ void coef_mm_d(const float* X, int ldx, int K,
                                          const float* __restrict__ W, int64_t dstride, int ldw,
                                          int Nout, int wave, int lane, floatx4 (&acc)[9][MAXJ]) {
  constexpr int NL = NC == 9 ? 3 : 1;
  const int ntile = Nout / 16;
  const int r = lane & 15, q = lane >> 4;
  // 32-bit element offsets from the (wave-uniform) weight base
  unsigned off[NL][MAXJ];
#pragma unroll
  for (int l = 0; l < NL; ++l)
#pragma unroll
    for (int jj = 0; jj < MAXJ; ++jj)
      off[l][jj] = (unsigned)(l * dstride + ((wave + NW * jj) % ntile) * 16 + r + 4 * q * ldw);
  auto loadb = [&](float (&b)[D][4][NL][MAXJ], int k0) {
#pragma unroll
    for (int d = 0; d < D; ++d)
#pragma unroll
      for (int s = 0; s < 4; ++s)
#pragma unroll
        for (int l = 0; l < NL; ++l)
#pragma unroll
          for (int jj = 0; jj < MAXJ; ++jj)
            b[d][s][l][jj] = W[off[l][jj] + (unsigned)((k0 + 16 * d + s) * ldw)];
  };
  const float* xr = X + r * ldx + 4 * q;
  auto mul = [&](const float (&b)[D][4][NL][MAXJ], int g0) {
#pragma unroll
    for (int d = 0; d < D; ++d) {
      const int k0 = g0 + 16 * d;
      floatx4 a[NC];
#pragma unroll
      for (int c = 0; c < NC; ++c)
        a[c] = *reinterpret_cast<const floatx4*>(xr + c * NT * ldx + k0);
#pragma unroll
      for (int s = 0; s < 4; ++s)
#pragma unroll
        for (int c = 0; c < NC; ++c)
#pragma unroll
          for (int jj = 0; jj < MAXJ; ++jj)
            acc[c][jj] = mfma4(a[c][s], b[d][s][NC == 9 ? ndeg(c) : 0][jj], acc[c][jj]);
    }
  };
  // two register buffers in turn: the next group's loads are in flight during this one's MFMAs
  constexpr int G = 16 * D;
  float b0[D][4][NL][MAXJ], b1[D][4][NL][MAXJ];
  loadb(b0, 0);
  for (int g0 = 0; g0 < K; g0 += 2 * G) {
    if (g0 + G < K) loadb(b1, g0 + G);
    mul(b0, g0);
    if (g0 + G >= K) break;
    if (g0 + 2 * G < K) loadb(b0, g0 + 2 * G);
    mul(b1, g0 + G);
  }
}

template <int NC>
__device__ __forceinline__ void coef_mm(const float* X, int ldx, int K,
                                        const float* __restrict__ W, int64_t dstride, int ldw,
                                        int Nout, int wave, int lane, floatx4 (&acc)[9][MAXJ]) {
  if (NC == 1 && K % 64 == 0)
    coef_mm_d<NC, 4>(X, ldx, K, W, dstride, ldw, Nout, wave, lane, acc);
  else
    coef_mm_d<NC, 1>(X, ldx, K, W, dstride, ldw, Nout, wave, lane, acc);
}

__device__ __forceinline__ void zero_acc(floatx4 (&acc)[9][MAXJ]) {
#pragma unroll
  for (int c = 0; c < 9; ++c)
#pragma unroll
    for (int jj = 0; jj < MAXJ; ++jj) acc[c][jj] = floatx4{0.f, 0.f, 0.f, 0.f};
}

// RMSNormSH forward of one node's 9 x C rows (norm.py:93-111): centre coefficient 0 over the
// channels, ms = mean_c sum_j bdw_j xc_j^2, inv = rsqrt(ms + eps), y = xc * inv * aw[l(j)],
// y[0] += ab (+ add0).  xs: the node's rows (stride xstride); writes y rows (stride ystride).
// One wavefront; lane handles channels lane, lane + 64.
__device__ __forceinline__ float rms_fwd_node(const float* xs, int64_t xstride, float* ys,
                                              int64_t ystride, const float* __restrict__ aw,
                                              const float* __restrict__ ab,
                                              const float* __restrict__ add0row, int C,
                                              int lane, float eps) {
  float s0 = 0.f;
  for (int c = lane; c < C; c += 64) s0 += xs[c];
  const float mu = tta_group_sum(s0, 64) / C;
  float ms = 0.f;
  for (int c = lane; c < C; c += 64) {
    float sc = 0.f;
#pragma unroll
    for (int j = 0; j < 9; ++j) {
      const float v = j == 0 ? xs[c] - mu : xs[j * xstride + c];
      sc += v * v * nbdw(j);
    }
    ms += sc;
  }
  ms = tta_group_sum(ms, 64) / C;
  const float inv = 1.0f / sqrtf(ms + eps);
  for (int c = lane; c < C; c += 64) {
    float v[9];
#pragma unroll
    for (int j = 0; j < 9; ++j) v[j] = j == 0 ? xs[c] - mu : xs[j * xstride + c];
#pragma unroll
    for (int j = 0; j < 9; ++j) {
      float o = v[j] * (inv * aw[ndeg(j) * C + c]);
      if (j == 0) {
        o = o + ab[c];
        if (add0row) o = o + add0row[c];
      }
      ys[j * ystride + c] = o;
    }
  }
  return inv;
}

// RMSNormSH backward of one node (forces.py:73-98): gx = g inv aw + xc bdw gms 2/C, minus the
// channel mean on coefficient 0.  gv(j, hh) / xv(j, hh) give the adjoint and the input of
// coefficient j at channel lane + 64 hh (registers or LDS, as the caller holds them); the
// results for those channels are returned in out[9][2].  The sums run over the lane's channels
// in order, then across the wavefront.
template <class GV, class XV>
__device__ __forceinline__ void rms_bwd_vals(GV gv, XV xv, const float* __restrict__ aw,
                                             float inv, int C, int lane, float (&out)[9][2]) {
  float s0 = 0.f;
#pragma unroll
  for (int hh = 0; hh < 2; ++hh)
    if (lane + 64 * hh < C) s0 += xv(0, hh);
  const float mu = tta_group_sum(s0, 64) / C;
  float ginv = 0.f;
#pragma unroll
  for (int hh = 0; hh < 2; ++hh) {
    const int c = lane + 64 * hh;
    if (c >= C) continue;
#pragma unroll
    for (int j = 0; j < 9; ++j) {
      const float v = j == 0 ? xv(0, hh) - mu : xv(j, hh);
      ginv += gv(j, hh) * v * aw[ndeg(j) * C + c];
    }
  }
  ginv = tta_group_sum(ginv, 64);
  const float gms = ginv * (inv * inv * inv) * -0.5f;
  float s1 = 0.f;
#pragma unroll
  for (int hh = 0; hh < 2; ++hh) {
    const int c = lane + 64 * hh;
    if (c >= C) continue;
    const float v = xv(0, hh) - mu;
    s1 += gv(0, hh) * (inv * aw[c]) + v * nbdw(0) * gms * (2.0f / C);
  }
  const float m0 = tta_group_sum(s1, 64) / C;
#pragma unroll
  for (int hh = 0; hh < 2; ++hh) {
    const int c = lane + 64 * hh;
#pragma unroll
    for (int j = 0; j < 9; ++j) {
      float gx = 0.f;
      if (c < C) {
        const float v = j == 0 ? xv(0, hh) - mu : xv(j, hh);
        gx = gv(j, hh) * (inv * aw[ndeg(j) * C + c]) + v * nbdw(j) * gms * (2.0f / C);
        if (j == 0) gx -= m0;
      }
      out[j][hh] = gx;
    }
  }
}

// The 16-node tile of a [N, 9, C] tensor into the [coefficient][node][channel] LDS layout, one
// wavefront per (node, coefficient) row (wave-uniform indices, no per-element division); rows
// of absent nodes are zero.
__device__ __forceinline__ void load_tile(float* buf, const float* __restrict__ x, int64_t n0,
                                          int nv, int C, int wave, int lane) {
  constexpr int RPW = 9 * NT / NW;   // rows per wave
  float v[RPW][2];                   // all of a wave's loads in flight before any store
#pragma unroll
  for (int i = 0; i < RPW; ++i) {
    const int rc = wave + NW * i, rr = rc / 9, c = rc - 9 * rr;
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      const int ch = lane + 64 * hh;
      v[i][hh] = (rr < nv && ch < C) ? x[((n0 + rr) * 9 + c) * C + ch] : 0.f;
    }
  }
#pragma unroll
  for (int i = 0; i < RPW; ++i) {
    const int rc = wave + NW * i, rr = rc / 9, c = rc - 9 * rr;
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      const int ch = lane + 64 * hh;
      if (ch < C) lrow(buf, c, rr)[ch] = v[i][hh];
    }
  }
}

struct SpecFwdArgs {
  const float* x1;                        // [N, 9, C] block state after the edgewise residual
  const float *aw2, *ab2;                 // norm_2 [3, C], [C]
  const float *ws_t, *bs;                 // scalar MLP [C, 2H], [2H]
  const float *w1t, *b1;                  // SO3_Linear_1 per degree [3, C, H], bias [H] (l = 0)
  const float *w2t, *b2;                  // SO3_Linear_2 per degree [3, H, C], bias [C] (l = 0)
  float *inv2, *a_s, *h;                  // saved: [N], [N, 2H] (pre-SiLU), [N, 9, H] (pre-gate)
  float* x2;                              // [N, 9, C] = x1 + FF
  const float *awn, *abn, *add0;          // next norm (may be null): [3, C], [C], [N, C] or null
  float *yn, *invn;                       // next norm output [N, 9, C], [N]
  int64_t N;
  int C, H;
  float eps;
  int npb;                                // nodes per workgroup, NT or NT / 2 (rows past it zero)
};

__global__ __launch_bounds__(NTH, 1) void k_spectral_block_fwd(SpecFwdArgs p) {
  __shared__ float buf[9 * NT * LDP];
  __shared__ float gat[NT * (2 * CMAX + 4)];
  const int t = threadIdx.x, lane = t & 63, wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int C = p.C, H = p.H, LH = 2 * H, ldg = 2 * CMAX + 4;
  const int64_t n0 = (int64_t)blockIdx.x * p.npb;
  const int nv = (int)min((int64_t)p.npb, p.N - n0);
  // 1. x1 rows -> LDS (rows of absent nodes zero)
  load_tile(buf, p.x1, n0, nv, C, wave, lane);
  __syncthreads();
  // 2. norm_2 in place, one wave per node
  for (int r = wave; r < nv; r += NW) {
    float* xs = lrow(buf, 0, r);
    const float inv = rms_fwd_node(xs, (int64_t)NT * LDP, xs, (int64_t)NT * LDP, p.aw2, p.ab2,
                                   nullptr, C, lane, p.eps);
    if (lane == 0) p.inv2[n0 + r] = inv;
  }
  __syncthreads();
  const int r = lane & 15, q = lane >> 4;
  floatx4 acc[9][MAXJ];
  // 3. scalar MLP on coefficient 0: a_s = n2_0 @ ws_t + bs (saved), gating = silu(a_s) -> LDS.
  //    2H columns = 2 x (H / 16) tiles; this wave takes tiles wave + NW jj of each H half.
#pragma unroll
  for (int half = 0; half < 2; ++half) {
    zero_acc(acc);
    coef_mm<1>(buf, LDP, C, p.ws_t + half * H, 0, LH, H, wave, lane, acc);
#pragma unroll
    for (int jj = 0; jj < MAXJ; ++jj) {
      const int j = wave + NW * jj;
      if (j >= H / 16) continue;
      const int col = half * H + j * 16 + r;
      const float bias = p.bs[col];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int row = 4 * q + e;
        const float a = acc[0][jj][e] + bias;
        if (row < nv) p.a_s[(n0 + row) * LH + col] = a;
        gat[row * ldg + col] = tta_silu(a);
      }
    }
  }
  // 4. h = n2 @ w1t[l] (+ b1 on coefficient 0)
  zero_acc(acc);
  coef_mm<9>(buf, LDP, C, p.w1t, (int64_t)C * H, H, H, wave, lane, acc);
  __syncthreads();  // every wave is done reading n2; gating is complete
  // 5. h saved; gout = gate(h) -> LDS (natural order: l = 1 rows gate block 0, l = 2 block 1);
  //    the gate values sigmoid(gating) once per (node, degree, channel)
  float sig[MAXJ][2][4];
#pragma unroll
  for (int jj = 0; jj < MAXJ; ++jj) {
    const int col = ((wave + NW * jj) % (H / 16)) * 16 + r;
#pragma unroll
    for (int l = 0; l < 2; ++l)
#pragma unroll
      for (int e = 0; e < 4; ++e)
        sig[jj][l][e] = tta_sigmoid_acc(gat[(4 * q + e) * ldg + l * H + col]);
  }
#pragma unroll
  for (int c = 0; c < 9; ++c)
#pragma unroll
    for (int jj = 0; jj < MAXJ; ++jj) {
      const int j = wave + NW * jj;
      if (j >= H / 16) continue;
      const int col = j * 16 + r;
      const float bias = c == 0 ? p.b1[col] : 0.f;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int row = 4 * q + e;
        const float v = acc[c][jj][e] + bias;
        if (row < nv) p.h[((n0 + row) * 9 + c) * H + col] = v;
        const float g = c == 0 ? tta_silu(v) : v * sig[jj][ndeg(c) - 1][e];
        lrow(buf, c, row)[col] = g;
      }
    }
  __syncthreads();
  // 6. out = x1 + gout @ w2t[l] (+ b2 on coefficient 0)
  zero_acc(acc);
  coef_mm<9>(buf, LDP, H, p.w2t, (int64_t)H * C, C, C, wave, lane, acc);
  if (p.awn) __syncthreads();  // the next norm reuses the buffer for x2
  // residual: all of this lane's x1 values are loaded before any x2 store, so the loads overlap
#pragma unroll
  for (int jj = 0; jj < MAXJ; ++jj) {
    const int j = wave + NW * jj;
    if (j >= C / 16) continue;
    const int col = j * 16 + r;
    const float b2 = p.b2[col];
    float xr[9][4];
#pragma unroll
    for (int c = 0; c < 9; ++c)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int row = 4 * q + e;
        xr[c][e] = row < nv ? p.x1[((n0 + row) * 9 + c) * C + col] : 0.f;
      }
#pragma unroll
    for (int c = 0; c < 9; ++c)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int row = 4 * q + e;
        const float v = acc[c][jj][e] + (c == 0 ? b2 : 0.f) + xr[c][e];
        if (row < nv) p.x2[((n0 + row) * 9 + c) * C + col] = v;
        if (p.awn) lrow(buf, c, row)[col] = v;
      }
  }
  if (!p.awn) return;
  __syncthreads();
  // 7. the next RMSNormSH on x2 (coefficient 0 + the system embedding when given)
  for (int rr = wave; rr < nv; rr += NW) {
    const int64_t n = n0 + rr;
    const float inv = rms_fwd_node(lrow(buf, 0, rr), (int64_t)NT * LDP, p.yn + n * 9 * C, C, p.awn,
                                   p.abn, p.add0 ? p.add0 + n * C : nullptr, C, lane, p.eps);
    if (lane == 0) p.invn[n] = inv;
  }
}

struct SpecBwdArgs {
  const float *g_n, *x2, *awn, *invn;     // next norm: output adjoint, input, weight, inv
  const float* res;                       // residual adjoint added to g_x2 (may be null)
  const float *x1, *aw2, *inv2, *a_s, *h; // this block's saved forward terms
  const float *w1, *w2, *ws;              // per degree [3, H, C], [3, C, H]; scalar [2H, C]
  float* g_x1;                            // [N, 9, C]
  int64_t N;
  int C, H;
  int npb;                                // nodes per workgroup, NT or NT / 2 (rows past it zero)
};

__global__ __launch_bounds__(NTH, 1) void k_spectral_block_bwd(SpecBwdArgs p) {
  __shared__ float buf[9 * NT * LDP];
  __shared__ float gas[NT * (2 * CMAX + 4)];
  const int t = threadIdx.x, lane = t & 63, wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int C = p.C, H = p.H, LH = 2 * H, ldg = 2 * CMAX + 4;
  const int64_t n0 = (int64_t)blockIdx.x * p.npb;
  const int nv = (int)min((int64_t)p.npb, p.N - n0);
  // 1. g_x2 = next-norm backward (+ res), one wave per node; kept in registers for step 5 and
  //    written to LDS as the FF's output adjoint (absent nodes: zero rows).  The x2 tile comes
  //    into LDS by coalesced rows; each wave's g_n values (its nodes wave + NW s, channels
  //    lane + 64 hh) go straight to registers, all loads in flight together.
  float gx2[NS][9][2];
  load_tile(buf, p.x2, n0, nv, C, wave, lane);
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    const int rr = wave + NW * s;
    const int64_t n = n0 + rr;
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      const int c = lane + 64 * hh;
      const bool in = rr < nv && c < C;
#pragma unroll
      for (int j = 0; j < 9; ++j) {
        gx2[s][j][hh] = in ? p.g_n[(n * 9 + j) * C + c] : 0.f;
      }
    }
  }
  __syncthreads();
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    const int rr = wave + NW * s;
    if (rr >= nv) {
      // an absent node's rows stay zero (its x2 rows were zero-filled above)
      continue;
    }
    const float* xs = lrow(buf, 0, rr);
    float o[9][2];
    rms_bwd_vals([&](int j, int hh) { return gx2[s][j][hh]; },
                 [&](int j, int hh) { return xs[j * NT * LDP + lane + 64 * hh]; }, p.awn,
                 p.invn[n0 + rr], C, lane, o);
    const int64_t n = n0 + rr;
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      const int c = lane + 64 * hh;
#pragma unroll
      for (int j = 0; j < 9; ++j) {
        gx2[s][j][hh] = o[j][hh] + ((p.res && c < C) ? p.res[(n * 9 + j) * C + c] : 0.f);
        if (c < C) lrow(buf, j, rr)[c] = gx2[s][j][hh];   // this wave's own node rows
      }
    }
  }
  __syncthreads();
  const int r = lane & 15, q = lane >> 4;
  floatx4 acc[9][MAXJ];
  // 2. g_gout = g_x2 @ w2[l]  ([C, H] per degree)
  zero_acc(acc);
  coef_mm<9>(buf, LDP, C, p.w2, (int64_t)C * H, H, H, wave, lane, acc);
  // 3. gate backward: g_h0 = g_gout0 silu'(h0); g_h_c = g_gout_c sig(gating); the degree sums
  //    sum_{c in l} g_gout_c h_c (register-local: this wave holds all nine coefficients of its
  //    columns) give g_a_s = sum * sig'(gating) * silu'(a_s)
  __syncthreads();  // every wave is done reading g_x2
#pragma unroll
  for (int jj = 0; jj < MAXJ; ++jj) {
    const int j = wave + NW * jj;
    if (j >= H / 16) continue;
    const int col = j * 16 + r;
    // this lane's saved forward values first (all loads in flight together)
    float hs[9][4], as[2][4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int row = 4 * q + e;
      const int64_t n = n0 + row;
      const bool in = row < nv;
#pragma unroll
      for (int c = 0; c < 9; ++c) hs[c][e] = in ? p.h[(n * 9 + c) * H + col] : 0.f;
      as[0][e] = in ? p.a_s[n * LH + col] : 0.f;
      as[1][e] = in ? p.a_s[n * LH + H + col] : 0.f;
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int row = 4 * q + e;
      float s1 = 0.f, s2 = 0.f;
      const float as1 = as[0][e], as2 = as[1][e];
      const float g1 = tta_silu(as1), g2 = tta_silu(as2);
      const float sg1 = tta_sigmoid_acc(g1), sg2 = tta_sigmoid_acc(g2);
#pragma unroll
      for (int c = 0; c < 9; ++c) {
        const float hv = hs[c][e];
        const float gg = acc[c][jj][e];
        float gh;
        if (c == 0) {
          gh = gg * tta_silu_grad(hv);
        } else if (c < 4) {
          gh = gg * sg1;
          s1 += gg * hv;
        } else {
          gh = gg * sg2;
          s2 += gg * hv;
        }
        lrow(buf, c, row)[col] = gh;
      }
      gas[row * ldg + col] = s1 * sg1 * (1.f - sg1) * tta_silu_grad(as1);
      gas[row * ldg + H + col] = s2 * sg2 * (1.f - sg2) * tta_silu_grad(as2);
    }
  }
  __syncthreads();
  // 4. g_n2 = g_h @ w1[l] ([H, C] per degree); coefficient 0 also + g_a_s @ ws ([2H, C]).  The
  //    x1 values step 5 needs are loaded first, so that they arrive during the products.
  float x1v[NS][9][2];
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    const int rr = wave + NW * s;
    const int64_t n = n0 + rr;
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      const int c = lane + 64 * hh;
#pragma unroll
      for (int j = 0; j < 9; ++j)
        x1v[s][j][hh] = (rr < nv && c < C) ? p.x1[(n * 9 + j) * C + c] : 0.f;
    }
  }
  zero_acc(acc);
  coef_mm<9>(buf, LDP, H, p.w1, (int64_t)H * C, C, C, wave, lane, acc);
  // + g_a_s @ ws on coefficient 0: the gas rows (stride ldg) as the A operand
  {
    floatx4 acc0[9][MAXJ];
    zero_acc(acc0);
    coef_mm<1>(gas, ldg, LH, p.ws, 0, C, C, wave, lane, acc0);
#pragma unroll
    for (int jj = 0; jj < MAXJ; ++jj) acc[0][jj] += acc0[0][jj];
  }
  __syncthreads();  // every wave is done reading g_h
#pragma unroll
  for (int c = 0; c < 9; ++c)
#pragma unroll
    for (int jj = 0; jj < MAXJ; ++jj) {
      const int j = wave + NW * jj;
      if (j >= C / 16) continue;
#pragma unroll
      for (int e = 0; e < 4; ++e) lrow(buf, c, 4 * q + e)[j * 16 + r] = acc[c][jj][e];
    }
  __syncthreads();
  // 5. g_x1 = norm_2 backward of g_n2 (LDS) with x1 from the registers loaded before step 4,
  //    plus g_x2
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    const int rr = wave + NW * s;
    if (rr >= nv) continue;
    const int64_t n = n0 + rr;
    const float* gs = lrow(buf, 0, rr);
    float gx[9][2];
    rms_bwd_vals([&](int j, int hh) { return gs[j * NT * LDP + lane + 64 * hh]; },
                 [&](int j, int hh) { return x1v[s][j][hh]; }, p.aw2, p.inv2[n], C, lane, gx);
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      const int c = lane + 64 * hh;
      if (c >= C) continue;
#pragma unroll
      for (int j = 0; j < 9; ++j) p.g_x1[(n * 9 + j) * C + c] = gx[j][hh] + gx2[s][j][hh];
    }
  }
}

struct HeadArgs {
  const float* ne;                        // final-norm output [N, 9, C] (coefficient 0 read)
  const float *w0t, *b0, *w1t, *b1, *w2, *b2;  // [C, H], [H], [H, H], [H], [H] (output row), [1]
  const float *w0, *w1;                   // backward: [H, C], [H, H] (torch [out, in])
  float *a1, *a2, *node_e;                // saved pre-activations [N, H] x 2, energies [N]
  float* g_ne;                            // backward output [N, 9, C]
  int64_t N;
  int C, H;
  int npb;                                // nodes per workgroup, NT or NT / 2 (rows past it zero)
};

// Per-node energy MLP on coefficient 0: a1 = ne0 @ w0t + b0, s1 = silu(a1), a2 = s1 @ w1t + b1,
// s2 = silu(a2), e = s2 . w2 + b2.
__global__ __launch_bounds__(NTH, 1) void k_energy_head_fwd(HeadArgs p) {
  __shared__ float buf[NT * LDP];
  const int t = threadIdx.x, lane = t & 63, wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int C = p.C, H = p.H;
  const int64_t n0 = (int64_t)blockIdx.x * p.npb;
  const int nv = (int)min((int64_t)p.npb, p.N - n0);
  for (int rr = wave; rr < NT; rr += NW)
    for (int ch = lane; ch < C; ch += 64)
      buf[rr * LDP + ch] = rr < nv ? p.ne[(n0 + rr) * 9 * C + ch] : 0.f;
  __syncthreads();
  const int r = lane & 15, q = lane >> 4;
  floatx4 acc[9][MAXJ];
  zero_acc(acc);
  coef_mm<1>(buf, LDP, C, p.w0t, 0, H, H, wave, lane, acc);
  __syncthreads();
#pragma unroll
  for (int jj = 0; jj < MAXJ; ++jj) {
    const int j = wave + NW * jj;
    if (j >= H / 16) continue;
    const int col = j * 16 + r;
    const float bias = p.b0[col];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int row = 4 * q + e;
      const float a = acc[0][jj][e] + bias;
      if (row < nv) p.a1[(n0 + row) * H + col] = a;
      buf[row * LDP + col] = tta_silu(a);
    }
  }
  __syncthreads();
  zero_acc(acc);
  coef_mm<1>(buf, LDP, H, p.w1t, 0, H, H, wave, lane, acc);
  __syncthreads();
#pragma unroll
  for (int jj = 0; jj < MAXJ; ++jj) {
    const int j = wave + NW * jj;
    if (j >= H / 16) continue;
    const int col = j * 16 + r;
    const float bias = p.b1[col];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int row = 4 * q + e;
      const float a = acc[0][jj][e] + bias;
      if (row < nv) p.a2[(n0 + row) * H + col] = a;
      buf[row * LDP + col] = tta_silu(a);
    }
  }
  __syncthreads();
  // e = s2 . w2 + b2: one wave per node, channels in order within each lane, then a butterfly
  for (int rr = wave; rr < nv; rr += NW) {
    float s = 0.f;
    for (int c = lane; c < H; c += 64) s += buf[rr * LDP + c] * p.w2[c];
    s = tta_group_sum(s, 64);
    if (lane == 0) p.node_e[n0 + rr] = s + p.b2[0];
  }
}

// dE/dnode_e = 1: g_a2 = w2 silu'(a2); g_a1 = (g_a2 @ w1) silu'(a1); g_ne0 = g_a1 @ w0; the
// other coefficients of g_ne are zero.
__global__ __launch_bounds__(NTH, 1) void k_energy_head_bwd(HeadArgs p) {
  __shared__ float buf[NT * LDP];
  const int t = threadIdx.x, lane = t & 63, wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int C = p.C, H = p.H;
  const int64_t n0 = (int64_t)blockIdx.x * p.npb;
  const int nv = (int)min((int64_t)p.npb, p.N - n0);
  for (int rr = wave; rr < NT; rr += NW)
    for (int ch = lane; ch < H; ch += 64)
      buf[rr * LDP + ch] = rr < nv ? p.w2[ch] * tta_silu_grad(p.a2[(n0 + rr) * H + ch]) : 0.f;
  __syncthreads();
  const int r = lane & 15, q = lane >> 4;
  floatx4 acc[9][MAXJ];
  zero_acc(acc);
  coef_mm<1>(buf, LDP, H, p.w1, 0, H, H, wave, lane, acc);
  __syncthreads();
#pragma unroll
  for (int jj = 0; jj < MAXJ; ++jj) {
    const int j = wave + NW * jj;
    if (j >= H / 16) continue;
    const int col = j * 16 + r;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int row = 4 * q + e;
      buf[row * LDP + col] =
          row < nv ? acc[0][jj][e] * tta_silu_grad(p.a1[(n0 + row) * H + col]) : 0.f;
    }
  }
  __syncthreads();
  zero_acc(acc);
  coef_mm<1>(buf, LDP, H, p.w0, 0, C, C, wave, lane, acc);
#pragma unroll
  for (int jj = 0; jj < MAXJ; ++jj) {
    const int j = wave + NW * jj;
    if (j >= C / 16) continue;
    const int col = j * 16 + r;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int row = 4 * q + e;
      if (row < nv) p.g_ne[(n0 + row) * 9 * C + col] = acc[0][jj][e];
    }
  }
  for (int rr = wave; rr < nv; rr += NW)
    for (int k = lane; k < 8 * C; k += 64) p.g_ne[(n0 + rr) * 9 * C + C + k] = 0.f;
}

bool node_dims_ok(int64_t N, int C, int H) {
  return N >= 0 && N < (1ll << 31) / 9 / 128 && C >= 16 && C <= CMAX && C % 16 == 0 &&
         H >= 16 && H <= CMAX && H % 16 == 0;
}

}  // namespace

// Nodes per workgroup of the node kernels: NT, or NT / 2 when NT-node workgroups would not
// cover the compute units (their MFMA tiles keep NT rows, the rows past the workgroup's nodes
// zero, so a half-full workgroup costs about what a full one does but the per-node phases --
// loads, norms, stores -- halve and twice as many units work).
static int spectral_npb(int64_t N) {
  // compute units per device, queried once; atomics, since host threads calling the library at
  // the same time may both fill an entry (with the same value)
  static std::atomic<int> cus_of[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
  int cus = cus_of[dev].load(std::memory_order_relaxed);
  if (cus == 0) {
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        cus <= 0)
      cus = 256;
    cus_of[dev].store(cus, std::memory_order_relaxed);
  }
  return (N + NT - 1) / NT < cus ? NT / 2 : NT;
}

extern "C" int tta_spectral_block_fwd(const float* x1, const float* aw2, const float* ab2,
                                      const float* ws_t, const float* bs, const float* w1t,
                                      const float* b1, const float* w2t, const float* b2,
                                      float* inv2, float* a_s, float* h, float* x2,
                                      const float* awn, const float* abn, const float* add0,
                                      float* yn, float* invn, int64_t N, int64_t C, int64_t H,
                                      float eps, hipStream_t stream) {
  TTA_CHECK_ARG(node_dims_ok(N, (int)C, (int)H),
                "tta_spectral_block_fwd: need C, H multiples of 16 in [16, 128] (got N=%lld C=%lld "
                "H=%lld)", (long long)N, (long long)C, (long long)H);
  TTA_CHECK_ARG(x1 && aw2 && ab2 && ws_t && bs && w1t && b1 && w2t && b2 && inv2 && a_s && h &&
                    x2,
                "tta_spectral_block_fwd: null pointer");
  TTA_CHECK_ARG(!awn || (abn && yn && invn), "tta_spectral_block_fwd: incomplete next norm");
  if (N == 0) return tta::kOk;
  SpecFwdArgs p{x1, aw2, ab2, ws_t, bs, w1t, b1, w2t, b2, inv2, a_s, h, x2,
                awn, abn, add0, yn, invn, N, (int)C, (int)H, eps, spectral_npb(N)};
  hipLaunchKernelGGL(k_spectral_block_fwd, dim3(tta_blocks(N, p.npb)), dim3(NTH), 0, stream, p);
  TTA_CHECK_LAUNCH("tta_spectral_block_fwd");
  return tta::kOk;
}

extern "C" int tta_spectral_block_bwd(const float* g_n, const float* x2, const float* awn,
                                      const float* invn, const float* res, const float* x1,
                                      const float* aw2, const float* inv2, const float* a_s,
                                      const float* h, const float* w1, const float* w2,
                                      const float* ws, float* g_x1, int64_t N, int64_t C,
                                      int64_t H, hipStream_t stream) {
  TTA_CHECK_ARG(node_dims_ok(N, (int)C, (int)H),
                "tta_spectral_block_bwd: need C, H multiples of 16 in [16, 128] (got N=%lld C=%lld "
                "H=%lld)", (long long)N, (long long)C, (long long)H);
  TTA_CHECK_ARG(g_n && x2 && awn && invn && x1 && aw2 && inv2 && a_s && h && w1 && w2 && ws &&
                    g_x1,
                "tta_spectral_block_bwd: null pointer");
  if (N == 0) return tta::kOk;
  SpecBwdArgs p{g_n, x2, awn, invn, res, x1, aw2, inv2, a_s, h, w1, w2, ws, g_x1, N, (int)C,
                (int)H, spectral_npb(N)};
  hipLaunchKernelGGL(k_spectral_block_bwd, dim3(tta_blocks(N, p.npb)), dim3(NTH), 0, stream, p);
  TTA_CHECK_LAUNCH("tta_spectral_block_bwd");
  return tta::kOk;
}

extern "C" int tta_energy_head_fwd(const float* ne, const float* w0t, const float* b0,
                                   const float* w1t, const float* b1, const float* w2,
                                   const float* b2, float* a1, float* a2, float* node_e,
                                   int64_t N, int64_t C, int64_t H, hipStream_t stream) {
  TTA_CHECK_ARG(node_dims_ok(N, (int)C, (int)H),
                "tta_energy_head_fwd: need C, H multiples of 16 in [16, 128]");
  TTA_CHECK_ARG(ne && w0t && b0 && w1t && b1 && w2 && b2 && a1 && a2 && node_e,
                "tta_energy_head_fwd: null pointer");
  if (N == 0) return tta::kOk;
  HeadArgs p{ne, w0t, b0, w1t, b1, w2, b2, nullptr, nullptr, a1, a2, node_e, nullptr, N, (int)C,
             (int)H, spectral_npb(N)};
  hipLaunchKernelGGL(k_energy_head_fwd, dim3(tta_blocks(N, p.npb)), dim3(NTH), 0, stream, p);
  TTA_CHECK_LAUNCH("tta_energy_head_fwd");
  return tta::kOk;
}

extern "C" int tta_energy_head_bwd(const float* a1, const float* a2, const float* w0,
                                   const float* w1, const float* w2, float* g_ne, int64_t N,
                                   int64_t C, int64_t H, hipStream_t stream) {
  TTA_CHECK_ARG(node_dims_ok(N, (int)C, (int)H),
                "tta_energy_head_bwd: need C, H multiples of 16 in [16, 128]");
  TTA_CHECK_ARG(a1 && a2 && w0 && w1 && w2 && g_ne, "tta_energy_head_bwd: null pointer");
  if (N == 0) return tta::kOk;
  HeadArgs p{nullptr, nullptr, nullptr, nullptr, nullptr, w2, nullptr, w0, w1,
             const_cast<float*>(a1), const_cast<float*>(a2), nullptr, g_ne, N, (int)C, (int)H,
             spectral_npb(N)};
  hipLaunchKernelGGL(k_energy_head_bwd, dim3(tta_blocks(N, p.npb)), dim3(NTH), 0, stream, p);
  TTA_CHECK_LAUNCH("tta_energy_head_bwd");
  return tta::kOk;
}
