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
//   mode 16: two fp16 planes each (v_mfma_f32_32x32x16_f16, same rate), three products
//           a0b0 + a0b1 + a1b0.  fp16 keeps 11 significant bits, so two planes hold 22 and the
//           dropped a1b1 and the plane roundings are ~2^-22 relative per product -- random in sign
//           and, summed over K, well below the fp32 accumulation error itself: fp32 GEMM accuracy
//           at half the MFMA work of mode 6.  fp16's 5-bit exponent needs scaling by powers of two
//           (exact): B column n by 2^-F[n] (F from the column's max |b|, packed after the planes),
//           A row r by 2^-E[r], E tracked online per 32-wide k slab.  E stays 0 while the row's
//           running max is in [2^-1, 2^15) (no scaling at all for ordinary activations); a k slab
//           whose values would reach 2^15 at the current E, or the row's first nonzero k slab
//           outside that window, resets E so the max lands below 2^11 and rescales the row's
//           accumulators by the (power-of-two) ratio.  Values far below the row max keep an
//           absolute error under 2^-24 of it (fp16 subnormals).  The epilogue multiplies each
//           accumulator by 2^(E[r] + F[n]).
//
// The 32x32x16 instruction: measured on MI355X it sustains about twice the bf16 rate of
// 16x16x32 (which issues at half rate).  Operand layout: lane l supplies A[l%32][8*(l/32) + e] and
// B[8*(l/32) + e][l%32], e = 0..7, of a 32 x 16 / 16 x 32 block.
//
// Packed B layout (tta_pack_b): bf16 [KT][planes][NT32][2][64 lanes][8] with KT = ceil(K/32) and
// NT32 padded to whole 128-column tiles: one 16(k) x 32(n) fragment is 1 KB, lane l holding
// B[kt*32 + ks*16 + 8*(l/32) + e][n32*32 + l%32] (zero beyond K, N).  Mode 16 stores fp16
// planes in the same order, followed by int32 F[NT32 * 32].
//
// Block tile (64 WM) x 128 x 32: WM x 2 waves, each 64 x 64 (2 x 2 MFMA tiles of 32 x 32); in
// mode 16, 2 WM waves of 32 x 128 (1 x 4 tiles), so that each A value split (the VALU work that
// bounds this mode) feeds four column tiles instead of two (+7 % over 64 x 64).  Both
// slabs of a k-step reach LDS by direct copies (buffer/global_load ... lds: lane i of a wave
// writes 16 bytes at the wave's LDS base + 16 i), with no register round trip: A as raw fp32 rows
// (16-byte chunks XOR-swizzled so that the fragment reads are conflict-free), B as packed.  The
// copies of slab kt+2 go into the stage slab kt leaves, right after the barrier that retires it,
// so they have a whole k-step to land.  Each wave reads its A fragment as fp32 (both 16-wide k
// halves of a slab at once, for mode 16's per-slab scale check) and splits it into planes in
// registers, one k half ahead of the MFMAs that consume it.  All modes run
// WM = 2: 128 x 128 tiles, 256 threads, 80 KB LDS (mode 6; 68 KB for mode 16, the epilogue's
// staging of the whole tile), so two blocks share a CU and one's
// epilogue, prologue and barriers overlap the other's MFMAs (measured faster than 256 x 128 tiles
// with one block per CU on every edge- and node-level shape of the two models).
#include "gemm_common.h"

#include <algorithm>
#include <atomic>

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __attribute__((address_space(3))) void* lds_ptr;
typedef __attribute__((address_space(1))) void* gbl_ptr;

namespace {

using namespace tta_gemm;

template <int MODE>
struct Split;
template <>
struct Split<1> {
  static constexpr int NA = 1, NB = 1, NP = 1;
  static constexpr bool F16 = false;
  static constexpr int pa[1] = {0};
  static constexpr int pb[1] = {0};
};
template <>
struct Split<3> {
  static constexpr int NA = 2, NB = 2, NP = 3;
  static constexpr bool F16 = false;
  static constexpr int pa[3] = {0, 1, 0};
  static constexpr int pb[3] = {1, 0, 0};
};
template <>
struct Split<6> {
  // smallest terms first
  static constexpr int NA = 3, NB = 3, NP = 6;
  static constexpr bool F16 = false;
  static constexpr int pa[6] = {1, 0, 2, 0, 1, 0};
  static constexpr int pb[6] = {1, 2, 0, 1, 0, 0};
};
template <>
struct Split<16> {
  static constexpr int NA = 2, NB = 2, NP = 3;
  static constexpr bool F16 = true;
  static constexpr int pa[3] = {1, 0, 0};
  static constexpr int pb[3] = {0, 1, 0};
};

// Fragment element type per plane format, and the 32x32x16 MFMA on it.
template <bool F16>
struct Frag {
  typedef bf16x8 T;
};
template <>
struct Frag<true> {
  typedef f16x8 T;
};
__device__ __forceinline__ floatx16 mfma32(bf16x8 a, bf16x8 b, floatx16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ floatx16 mfma32(f16x8 a, f16x8 b, floatx16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// mode 16 scaling: a B column's values are multiplied by 2^-(e - kTop), e the frexp exponent of
// its max |value| (max < 2^e), so they land below 2^kTop; an A row's shift follows the rule in the
// header.  kNoExp marks an A row with no nonzero value yet.
constexpr int kTop = 11, kNoExp = -100000;

constexpr int BN = 128, BK = 32;
constexpr int NF = (BN / 32) * 2;  // B fragments per plane per k-step: n32 tiles x k16 halves

__device__ __forceinline__ float epi_one(const GemmArgs& p, float v, int row, int col) {
  if (p.bias) v += p.bias[col];
  if (p.P)
    v += p.P[(int64_t)p.idx0[row] * p.ldp + col] + p.P[(int64_t)p.idx1[row] * p.ldp + p.off1 + col];
  const int64_t off = (int64_t)row * p.ldc + col;
  if (p.epi == EPI_SILU) v = tta_silu(v);
  if (p.epi == EPI_SIGMOID) v = tta_sigmoid_acc(v);
  if (p.epi == EPI_ACCUM) v += p.C[off];
  if (p.epi == EPI_PRE_SILU) p.C2[off] = tta_silu(v);
  if (p.epi == EPI_SILU_GRAD) v = v * tta_silu_grad(p.aux[off]);
  return v;
}

// Rows [row0, row0 + rows) of a 128-column output tile staged in LDS (row stride ldt floats).
// Thread t owns float4 column group t % 32 and rows t / 32, t / 32 + nth / 32, ...: the bias,
// the column checks and the lane's column offset are set once, and the epilogue type is a
// template parameter, so a row costs one LDS read, one address add and one 16-byte store.
// vec_ok (host-checked 16-byte alignment of every operand row) selects the float4 path; full
// (the tile lies inside M x N) drops the bounds checks.
// Split-K: rows [row0, row0 + rows) of a staged tile, as they are, into the chunk's partial W
// (row-major, row stride N, 16-byte aligned base); the reduction applies bias and epilogue.
__device__ __forceinline__ void partial_rows(float* W, int M, int N, const float* Ct, int ldt,
                                             int rows, int row0, int n0, int t, int nth) {
  const int c4 = t & 31, rstep = nth >> 5;
  const int col = n0 + 4 * c4;
  if (col >= N) return;
  for (int rr = t >> 5; rr < rows; rr += rstep) {
    const int row = row0 + rr;
    if (row >= M) break;
    const floatx4 a = *reinterpret_cast<const floatx4*>(Ct + rr * ldt + 4 * c4);
    float* w = W + (int64_t)row * N + col;
    if (N % 4 == 0 && col + 3 < N) {
      *reinterpret_cast<floatx4*>(w) = a;
    } else {
      for (int e = 0; e < 4 && col + e < N; ++e) w[e] = a[e];
    }
  }
}

// EPI_GATE / EPI_GATE_BWD (ge, gc0: the launch's gate operands and the product's first
// coefficient) take the float4 path only (the host requires their alignments); a thread's four
// columns lie in one coefficient (H % 4 == 0).
template <int EPI, bool BATCH>
__device__ __forceinline__ void epilogue_rows(const GemmArgs& p, const float* Ct, int ldt,
                                              int rows, int row0, int n0, int t, int nth,
                                              bool vec_ok, bool full,
                                              const GateEpi* ge = nullptr, int gc0 = 0) {
  constexpr bool GATE = EPI == EPI_GATE || EPI == EPI_GATE_BWD;
  const int c4 = t & 31, rstep = nth >> 5;
  const int col = n0 + 4 * c4;
  if (vec_ok && (full || col + 3 < p.N)) {
    const floatx4 bv = p.bias ? *reinterpret_cast<const floatx4*>(p.bias + col)
                              : floatx4{0.f, 0.f, 0.f, 0.f};
    const bool gather = p.P != nullptr;
    // gate: coefficient gc of this thread's columns, their channel gh, gating column gcol
    int gc = 0, gh = 0, gcol = 0;
    if constexpr (GATE) {
      gc = gate_coef(*ge, gc0, col);
      gh = col - (gc - gc0) * ge->H;
      gcol = gc > 0 ? gate_gcol(*ge, gc, gh) : 0;
    }
    // gate epilogue of one float4: coefficient 0 stores its pre-activation and takes SiLU (the
    // backward: is multiplied by silu' of the stored x0 values gv), the others are scaled by their
    // gating sigmoids gv
    auto gate4 = [&](floatx4& v, const floatx4& gv, int row) {
      if (gc > 0) {
        v = v * gv;
      } else if constexpr (EPI == EPI_GATE) {
        __builtin_nontemporal_store(v, reinterpret_cast<floatx4*>(ge->x0 + (int64_t)row * ge->ldx0 + gh));
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = tta_silu(v[e]);
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = v[e] * tta_silu_grad(gv[e]);
      }
    };
    // the gate operand of one float4 of row `row`: its sigmoids, or (backward, coefficient 0) x0
    auto gload = [&](int row) -> floatx4 {
      if (gc > 0)
        return *reinterpret_cast<const floatx4*>(ge->sig + (int64_t)row * ge->ldg + gcol);
      if constexpr (EPI == EPI_GATE_BWD)
        return *reinterpret_cast<const floatx4*>(ge->x0 + (int64_t)row * ge->ldx0 + gh);
      return floatx4{0.f, 0.f, 0.f, 0.f};
    };
    constexpr bool LOADS = EPI == EPI_ACCUM || EPI == EPI_SILU_GRAD || GATE;
    constexpr int RB = 8;
    if (BATCH && full && (LOADS || gather) && rows % (RB * rstep) == 0) {
      // An epilogue that reads memory (the accumulated C, the SiLU argument, the gathered rows;
      // BATCH: mode 16, whose register budget has room for it)
      // issues a batch of RB rows' loads -- the gather indices first, then the rows they name --
      // before it uses any, so their latencies overlap instead of adding up row by row.
#pragma unroll 1
      for (int rb = t >> 5; rb < rows; rb += RB * rstep) {
        int i0[RB], i1[RB];
        floatx4 ex[RB], pv[RB];
#pragma unroll
        for (int i = 0; i < RB; ++i) {
          const int row = row0 + rb + i * rstep;
          if (gather) {
            i0[i] = p.idx0[row];
            i1[i] = p.idx1[row];
          }
          if constexpr (EPI == EPI_ACCUM)
            ex[i] = *reinterpret_cast<const floatx4*>(p.C + (int64_t)row * p.ldc + col);
          if constexpr (EPI == EPI_SILU_GRAD)
            ex[i] = *reinterpret_cast<const floatx4*>(p.aux + (int64_t)row * p.ldc + col);
          if constexpr (GATE) ex[i] = gload(row);
        }
        if (gather) {
#pragma unroll
          for (int i = 0; i < RB; ++i)
            pv[i] = *reinterpret_cast<const floatx4*>(p.P + (int64_t)i0[i] * p.ldp + col) +
                    *reinterpret_cast<const floatx4*>(p.P + (int64_t)i1[i] * p.ldp + p.off1 + col);
        }
#pragma unroll
        for (int i = 0; i < RB; ++i) {
          const int rr = rb + i * rstep, row = row0 + rr;
          floatx4 v = *reinterpret_cast<const floatx4*>(Ct + rr * ldt + 4 * c4) + bv;
          const int64_t off = (int64_t)row * p.ldc + col;
          if (gather) v += pv[i];
          if constexpr (EPI == EPI_ACCUM) v += ex[i];
          if constexpr (GATE) gate4(v, ex[i], row);
          if constexpr (EPI == EPI_SIGMOID) {
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] = tta_sigmoid_acc(v[e]);
          }
          if constexpr (EPI == EPI_SILU || EPI == EPI_PRE_SILU || EPI == EPI_SILU_GRAD) {
            floatx4 w;
#pragma unroll
            for (int e = 0; e < 4; ++e)
              w[e] = EPI == EPI_SILU_GRAD ? v[e] * tta_silu_grad(ex[i][e]) : tta_silu(v[e]);
            if constexpr (EPI == EPI_PRE_SILU)
              __builtin_nontemporal_store(w, reinterpret_cast<floatx4*>(p.C2 + off));
            else
              v = w;
          }
          __builtin_nontemporal_store(v, reinterpret_cast<floatx4*>(p.C + off));
        }
      }
      return;
    }
#pragma unroll 4
    for (int rr = t >> 5; rr < rows; rr += rstep) {
      const int row = row0 + rr;
      if (!full && row >= p.M) break;
      floatx4 v = *reinterpret_cast<const floatx4*>(Ct + rr * ldt + 4 * c4) + bv;
      const int64_t off = (int64_t)row * p.ldc + col;
      if (gather)
        v += *reinterpret_cast<const floatx4*>(p.P + (int64_t)p.idx0[row] * p.ldp + col) +
             *reinterpret_cast<const floatx4*>(p.P + (int64_t)p.idx1[row] * p.ldp + p.off1 + col);
      if constexpr (EPI == EPI_ACCUM) v += *reinterpret_cast<const floatx4*>(p.C + off);
      if constexpr (GATE) gate4(v, gload(row), row);
      if constexpr (EPI == EPI_SIGMOID) {
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = tta_sigmoid_acc(v[e]);
      }
      if constexpr (EPI == EPI_SILU || EPI == EPI_PRE_SILU || EPI == EPI_SILU_GRAD) {
        floatx4 w;
        if constexpr (EPI == EPI_SILU_GRAD) {
          const floatx4 x = *reinterpret_cast<const floatx4*>(p.aux + off);
#pragma unroll
          for (int e = 0; e < 4; ++e) w[e] = v[e] * tta_silu_grad(x[e]);
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e) w[e] = tta_silu(v[e]);
        }
        if constexpr (EPI == EPI_PRE_SILU)
          __builtin_nontemporal_store(w, reinterpret_cast<floatx4*>(p.C2 + off));
        else
          v = w;
      }
      // streaming stores: the outputs (hundreds of MB on edge-level shapes) would otherwise
      // evict the A row panels that the other column tiles are still re-reading from L2
      // (+15-17 % on the write-heavy short-K shapes)
      __builtin_nontemporal_store(v, reinterpret_cast<floatx4*>(p.C + off));
    }
  } else if constexpr (!GATE) {
    for (int rr = t >> 5; rr < rows; rr += rstep) {
      const int row = row0 + rr;
      if (row >= p.M) break;
      const floatx4 a = *reinterpret_cast<const floatx4*>(Ct + rr * ldt + 4 * c4);
      for (int e = 0; e < 4 && col + e < p.N; ++e)
        p.C[(int64_t)row * p.ldc + col + e] = epi_one(p, a[e], row, col + e);
    }
  }
}

// Split 8 fp32 values into NPL bf16 planes (round-to-nearest residuals), pairs at a time.
template <int NPL>
__device__ __forceinline__ void split8(const floatx4& x0, const floatx4& x1, bf16x8 (&out)[NPL]) {
  typedef float f2 __attribute__((ext_vector_type(2)));
  typedef __bf16 h2 __attribute__((ext_vector_type(2)));
  f2 r[4] = {f2{x0[0], x0[1]}, f2{x0[2], x0[3]}, f2{x1[0], x1[1]}, f2{x1[2], x1[3]}};
#pragma unroll
  for (int q = 0; q < NPL; ++q) {
    h2 h[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      h[i] = __builtin_convertvector(r[i], h2);
      if (q + 1 < NPL) r[i] = r[i] - __builtin_convertvector(h[i], f2);
    }
    out[q] = bf16x8{h[0][0], h[0][1], h[1][0], h[1][1], h[2][0], h[2][1], h[3][0], h[3][1]};
  }
}

// x - (fp16 half 0 / half 1 of hpair) in one v_fma_mix_f32, which reads the fp16 operand in
// place (op_sel_hi marks source 0 as fp16, op_sel picks its half): no conversion back to fp32.
__device__ __forceinline__ float resid_lo(float x, unsigned hpair) {
  float r;
  asm("v_fma_mix_f32 %0, %1, -1.0, %2 op_sel_hi:[1,0,0]" : "=v"(r) : "v"(hpair), "v"(x));
  return r;
}
__device__ __forceinline__ float resid_hi(float x, unsigned hpair) {
  float r;
  asm("v_fma_mix_f32 %0, %1, -1.0, %2 op_sel:[1,0,0] op_sel_hi:[1,0,0]"
      : "=v"(r)
      : "v"(hpair), "v"(x));
  return r;
}

// max(|a|, |b|, c) and max(a, b, c) in one v_max3_f32 (abs as source modifiers; fmaxf would
// add a canonicalising max per operand).  Only the exponent of the result is used.
__device__ __forceinline__ float max3_abs(float a, float b, float c) {
  float r;
  asm("v_max3_f32 %0, |%1|, |%2|, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
  return r;
}
__device__ __forceinline__ float max3(float a, float b, float c) {
  float r;
  asm("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
  return r;
}

// Split 8 fp32 values, scaled by 2^-sh, into two fp16 planes (round-to-nearest residuals).
template <int NPL>
__device__ __forceinline__ void split8_f16(const floatx4& x0, const floatx4& x1, int sh,
                                           f16x8 (&out)[NPL]) {
  static_assert(NPL == 2, "two fp16 planes");
  typedef float f2 __attribute__((ext_vector_type(2)));
  typedef _Float16 h2 __attribute__((ext_vector_type(2)));
  f2 r[4];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    r[i] = f2{__builtin_amdgcn_ldexpf(x0[2 * i], -sh), __builtin_amdgcn_ldexpf(x0[2 * i + 1], -sh)};
    r[i + 2] =
        f2{__builtin_amdgcn_ldexpf(x1[2 * i], -sh), __builtin_amdgcn_ldexpf(x1[2 * i + 1], -sh)};
  }
  h2 h[4], l[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    h[i] = __builtin_convertvector(r[i], h2);
    const unsigned hp = __builtin_bit_cast(unsigned, h[i]);
    l[i] = __builtin_convertvector(f2{resid_lo(r[i][0], hp), resid_hi(r[i][1], hp)}, h2);
  }
  out[0] = f16x8{h[0][0], h[0][1], h[1][0], h[1][1], h[2][0], h[2][1], h[3][0], h[3][1]};
  out[1] = f16x8{l[0][0], l[0][1], l[1][0], l[1][1], l[2][0], l[2][1], l[3][0], l[3][1]};
}

// A (fp32) tile row: 8 chunks of 16 B per 32-wide k slab, chunk c of row r stored at c ^ aswz(r):
// 16 consecutive rows at one logical chunk then cover all 64 banks.
__device__ __forceinline__ int aswz(int row) { return (row >> 1) & 7; }

template <int WM, int MODE>
__global__ __launch_bounds__(128 * WM, WM == 2 ? 2 : 1) void gemm_bf16x_kernel(GemmGroup g) {
  const GemmArgs& p = g.p[blockIdx.z];  // the product of this block (group of one: z = 0)
  const int K = p.K;                     // kept in a scalar register across the k loop
  const int NT32 = g.NT32[blockIdx.z];
  const bool vec_ok = g.vec[blockIdx.z] != 0;
  typedef Split<MODE> S;
  // wave tile: TI row blocks x TJ column blocks of 32 x 32 (mode 16: 32 x 128, one A split feeds
  // four column blocks)
  constexpr int TI = S::F16 ? 1 : 2, TJ = 4 / TI;
  typedef typename Frag<S::F16>::T V8;
  constexpr int NA = S::NA, NB = S::NB;
  constexpr int BM = 64 * WM, NTH = 128 * WM;
  constexpr int A_CH = BM * 8, B_CH = NB * NF * 64, STG = A_CH + B_CH;  // 16-byte chunks
  constexpr int APT = A_CH / NTH, BPT = B_CH / NTH;                      // copies per thread
  static_assert(APT * NTH == A_CH && BPT * NTH == B_CH, "slabs must split evenly");
  // two slab stages; mode 16 (64 KB of stages) rounds up to the whole output tile, 68 KB, for a
  // one-pass epilogue at the same two blocks per CU (modes 1 and 3 keep 48 / 64 KB: three blocks
  // per CU for mode 1)
  constexpr int LDT = BN + 8;
  constexpr int SMEM_U4 = (S::F16 && BM * LDT / 4 > 2 * STG) ? BM * LDT / 4 : 2 * STG;
  __shared__ uint4 smem[SMEM_U4];

  const int t = threadIdx.x;
  const int lane = t & 63;
  const int wave = t >> 6;
  const int wm = TI == 2 ? wave >> 1 : wave, wn = TI == 2 ? wave & 1 : 0;
  const int tn = (p.N + BN - 1) / BN;
  const int ntiles = tn * ((p.M + BM - 1) / BM);
  // Persistent tiles: a product of a group runs on the first gb = min(ntiles rounded up to 8,
  // g.cap) blocks of the grid (wider grids belong to other products).  Block b sits on XCD b % 8
  // (the dispatcher's round robin) and walks that XCD's contiguous range of tiles -- row-major
  // (m, n) order, so neighbours share A row panels in that XCD's L2 -- with stride gb / 8.
  const int gb = min(((ntiles + 7) / 8) * 8, g.cap);
  if ((int)blockIdx.x >= gb) return;
  const int per_xcd = (ntiles + 7) / 8, stride = gb / 8;
  const int t_end = min(((int)blockIdx.x % 8 + 1) * per_xcd, ntiles);
  int tile = ((int)blockIdx.x % 8) * per_xcd + (int)blockIdx.x / 8;
  if (tile >= t_end) return;
  const uint4* Bp = static_cast<const uint4*>(p.B);
  // Copy offsets: the per-lane byte offsets are fixed for a tile and the k step enters as the
  // (scalar) soffset, so a k step's copies cost no vector address arithmetic.  A goes through a
  // buffer resource based at the tile's first row; a row past M gets a voffset past num_records
  // (copied as zeros); a slab that runs past K (K % 32 != 0, the last slab only) checks its
  // columns per lane instead.  LDS destinations are wave-uniform.
  const int wave_s = __builtin_amdgcn_readfirstlane(wave);
  int arow[APT], aoff[APT], acol[APT];
#pragma unroll
  for (int h = 0; h < APT; ++h) {
    const int L = t + NTH * h;  // LDS chunk this lane fills
    arow[h] = L >> 3;
    acol[h] = 4 * ((L & 7) ^ aswz(arow[h]));
    aoff[h] = (arow[h] * (int)p.lda + acol[h]) * 4;
  }
  // packed B: every offset of the buffer fits in 31 bits (checked on the host)
  const __amdgpu_buffer_rsrc_t brsrc =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p.B), (short)0, 0x7ffffffe, 0x00020000);
  int boff[BPT];
#pragma unroll
  for (int h = 0; h < BPT; ++h) {
    const int c = t + NTH * h;
    const int pl = c / (NF * 64), f = (c / 64) % NF, l = c % 64;
    boff[h] = (((pl * NT32 + (f >> 1)) * 2 + (f & 1)) * 64 + l) * 16;
  }
  const int bstep = NB * NT32 * 128 * 16;  // bytes of one packed k slab

  // copy parameters of the tile being loaded: they move on to the next tile after the epilogue's
  // last lgkmcnt(0) + s_barrier, and only then are that tile's slab-0 copies issued, because the
  // epilogue's staging area aliases stage 0
  int m0 = 0, n0 = 0;
  __amdgpu_buffer_rsrc_t arsrc;
  int avo[APT], bvo[BPT];
  auto set_tile = [&](int tl) {
    n0 = (tl % tn) * BN;
    m0 = (tl / tn) * BM;
    arsrc = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(p.A + (int64_t)m0 * p.lda),
                                              (short)0, 0x7ffffffe, 0x00020000);
    const int rows_left = p.M - m0;
#pragma unroll
    for (int h = 0; h < APT; ++h) avo[h] = arow[h] < rows_left ? aoff[h] : (int)0x7fffffff;
#pragma unroll
    for (int h = 0; h < BPT; ++h) bvo[h] = boff[h] + (n0 / 32) * 2048;
  };

  auto issue = [&](int kt, int stg) {
    uint4* base = smem + stg * STG + 64 * wave_s;  // + NTH * h: this wave's 64 chunks of copy h
    const int k0 = kt * BK;
    // (the offsets go through locals: hipcc's host pass drops the kernel's launch stub when a
    // builtin argument reads a lambda-captured array element directly)
    if (k0 + BK <= K) {
#pragma unroll
      for (int h = 0; h < APT; ++h) {
        const int vo = avo[h];
        __builtin_amdgcn_raw_ptr_buffer_load_lds(arsrc, (lds_ptr)(base + NTH * h), 16, vo,
                                                 k0 * 4, 0, 0);
      }
    } else {
#pragma unroll
      for (int h = 0; h < APT; ++h) {
        const int vo = avo[h], k = k0 + acol[h];
        const int off = (vo != (int)0x7fffffff && k < K) ? vo + k0 * 4 : (int)0x7fffffff;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(arsrc, (lds_ptr)(base + NTH * h), 16, off, 0, 0,
                                                 0);
      }
    }
#pragma unroll
    for (int h = 0; h < BPT; ++h) {
      const int vo = bvo[h];
      __builtin_amdgcn_raw_ptr_buffer_load_lds(brsrc, (lds_ptr)(base + A_CH + NTH * h), 16, vo,
                                               kt * bstep, 0, 0);
    }
  };
  // the copies of a slab that ends inside K (every slab when K % 32 == 0): no column checks
  auto issue_full = [&](int kt, int stg) {
    uint4* base = smem + stg * STG + 64 * wave_s;
#pragma unroll
    for (int h = 0; h < APT; ++h) {
      const int vo = avo[h];
      __builtin_amdgcn_raw_ptr_buffer_load_lds(arsrc, (lds_ptr)(base + NTH * h), 16, vo,
                                               kt * BK * 4, 0, 0);
    }
#pragma unroll
    for (int h = 0; h < BPT; ++h) {
      const int vo = bvo[h];
      __builtin_amdgcn_raw_ptr_buffer_load_lds(brsrc, (lds_ptr)(base + A_CH + NTH * h), 16, vo,
                                               kt * bstep, 0, 0);
    }
  };

  floatx16 acc[TI][TJ];
#pragma unroll
  for (int i = 0; i < TI; ++i)
#pragma unroll
    for (int j = 0; j < TJ; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  const int l32 = lane & 31, lh = lane >> 5;
  const int rbase = wm * 32 * TI, cbase = wn * 32 * TJ;
  // Fragment reads of one 16-wide k half: raw fp32 A (split later) and the packed B planes.
  auto rdB = [&](int stg, int ks, V8 (&b)[TJ][NB]) {
    const uint4* Bs = smem + stg * STG + A_CH;
#pragma unroll
    for (int j = 0; j < TJ; ++j)
#pragma unroll
      for (int q = 0; q < NB; ++q)
        b[j][q] = __builtin_bit_cast(V8, Bs[(q * NF + (wn * TJ + j) * 2 + ks) * 64 + lane]);
  };
  auto rdA = [&](int stg, int ks, floatx4 (&x)[TI][2]) {
    const uint4* As = smem + stg * STG;
#pragma unroll
    for (int i = 0; i < TI; ++i) {
      const int row = rbase + i * 32 + l32;
      const int c0 = 4 * ks + 2 * lh;
      x[i][0] = __builtin_bit_cast(floatx4, As[row * 8 + (c0 ^ aswz(row))]);
      x[i][1] = __builtin_bit_cast(floatx4, As[row * 8 + ((c0 + 1) ^ aswz(row))]);
    }
  };
  // mode 16: er[i] = shift E of the lane's A row l32 of row block i, whose values enter the
  // planes multiplied by 2^-E (lanes l and l + 32 hold the same row and agree); accumulator
  // element r of a 32 x 32 block belongs to row crow(r) of the block, whose shift lane crow(r)
  // holds.  The shift is checked once per 32-wide k slab, over both of its halves.
  int er[TI];
#pragma unroll
  for (int i = 0; i < TI; ++i) er[i] = kNoExp;
  bool unscaled = true;  // wave-uniform: E is 0 or unset on every row (the common case)
  auto crow = [&](int r) { return 8 * (r >> 2) + 4 * lh + (r & 3); };
  // returns whether a shift changed (the accumulators were rescaled)
  auto scale = [&](const floatx4 (&x0)[TI][2], const floatx4 (&x1)[TI][2]) -> bool {
    if constexpr (S::F16) {
      int en[TI];
      bool grow = false;
#pragma unroll
      for (int i = 0; i < TI; ++i) {
        float m = 0.f;
#pragma unroll
        for (int c = 0; c < 2; ++c)
#pragma unroll
          for (int e = 0; e < 4; ++e) m = max3_abs(x0[i][c][e], x1[i][c][e], m);
        // the row's other 16 values of this k slab are in lane l ^ 32: v_permlane32_swap trades
        // the upper half of one register with the lower half of another, so with m in both, one
        // of them ends up holding the partner's m in every lane (a permute through LDS would wait
        // on the fragment reads in flight).  s_nop 1: the two wait states the swap needs after
        // the VALU writes of its operands.
        {
          float u = m, w = m;
          asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(u), "+v"(w));
          m = max3(m, u, w);
        }
        const int e = m > 0.f ? __builtin_amdgcn_frexp_expf(m) : kNoExp;
        // values below 2^e reach 2^(e - E): a new shift once that passes 2^15, and for the row's
        // first nonzero slab (E = kNoExp); the new shift is never below the old one
        const bool g = e != kNoExp && e - er[i] > 15;
        en[i] = g ? ((e >= 0 && e <= 15) ? 0 : e - kTop) : er[i];
        grow |= g;
      }
      if (__any(grow)) {  // rare: a row's first nonzero k slab, or a much larger value
#pragma unroll
        for (int i = 0; i < TI; ++i) {
          const int d = er[i] - en[i];  // <= 0; the sentinel's huge d zeroes an all-zero acc
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int dr = __shfl(d, crow(r));
#pragma unroll
            for (int j = 0; j < TJ; ++j) acc[i][j][r] = __builtin_amdgcn_ldexpf(acc[i][j][r], dr);
          }
          er[i] = en[i];
        }
        bool u = true;
#pragma unroll
        for (int i = 0; i < TI; ++i) u &= er[i] == 0 || er[i] == kNoExp;
        unscaled = __all(u);
        return true;
      }
    }
    return false;
  };
  // the split of an unscaled wave (every mode but a scaled mode-16 wave): no branch, so that the
  // scheduler can interleave it with the MFMAs of the other k half
  auto sp_fast = [&](const floatx4 (&x)[TI][2], V8 (&a)[TI][NA]) {
#pragma unroll
    for (int i = 0; i < TI; ++i) {
      if constexpr (S::F16)
        split8_f16<NA>(x[i][0], x[i][1], 0, a[i]);
      else
        split8<NA>(x[i][0], x[i][1], a[i]);
    }
  };
  auto sp = [&](const floatx4 (&x)[TI][2], V8 (&a)[TI][NA]) {
    if constexpr (S::F16) {
      // E = 0 on every row of the wave (the common case): no scaling instructions at all
      if (unscaled) {
#pragma unroll
        for (int i = 0; i < TI; ++i) split8_f16<NA>(x[i][0], x[i][1], 0, a[i]);
      } else {
#pragma unroll
        for (int i = 0; i < TI; ++i) split8_f16<NA>(x[i][0], x[i][1], er[i], a[i]);
      }
    } else {
#pragma unroll
      for (int i = 0; i < TI; ++i) split8<NA>(x[i][0], x[i][1], a[i]);
    }
  };
  auto mm = [&](const V8 (&a)[TI][NA], const V8 (&b)[TJ][NB]) {
#pragma unroll
    for (int q = 0; q < S::NP; ++q)
#pragma unroll
      for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int j = 0; j < TJ; ++j) acc[i][j] = mfma32(a[i][S::pa[q]], b[j][S::pb[q]], acc[i][j]);
  };

  // Software pipeline: the fragments of the next k half are read (and A split) while the MFMAs of
  // the current one run.  One barrier per slab: each wave arrives with its copies of slab kt+1
  // landed and its reads of slab kt returned, so after it slab kt+1 is visible to all and slab kt's
  // stage takes the copies of slab kt+2.  Slab indices past the end are clamped (harmless
  // re-copies, never read) so every step issues the same copies.  A tile's slab 0 always sits in
  // stage 0, slab 1 in stage 1.
  const int nk = (K + BK - 1) / BK;
  // k range of this block: slabs [kt0, kt1), all of K, or with split-K (g.work set) chunk
  // blockIdx.y of g.kch[z] columns (a multiple of BK), whose partial product goes to g.work
  const bool split = g.work != nullptr;
  const int kt0 = split ? (int)blockIdx.y * (g.kch[blockIdx.z] / BK) : 0;
  const int kt1 = split ? min(nk, kt0 + g.kch[blockIdx.z] / BK) : nk;
  if (kt0 >= kt1 && split) return;
  const int* Fc =
      S::F16 ? reinterpret_cast<const int*>(Bp + (int64_t)nk * NB * NT32 * 128) : nullptr;
  constexpr int SMEM_F = SMEM_U4 * 4;
  constexpr int RP = (BM * LDT <= SMEM_F) ? BM : (BM / 2 * LDT <= SMEM_F) ? BM / 2
                   : (BM / 4 * LDT <= SMEM_F) ? BM / 4 : 32;
  static_assert(RP % 32 == 0 && RP * LDT <= SMEM_F, "epilogue staging must fit the LDS buffer");

  set_tile(tile);
  if (kt1 > kt0) issue(kt0, 0);
  for (;;) {
    const int cm0 = m0, cn0 = n0;  // the tile computed in this pass
#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
      for (int j = 0; j < TJ; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;
#pragma unroll
    for (int i = 0; i < TI; ++i) er[i] = kNoExp;
    unscaled = true;
    if (kt1 > kt0) {
      issue(min(kt0 + 1, kt1 - 1), 1);
      // slab 0 landed (with everything issued before it: vector memory operations complete in
      // order); slab 1 may still be in flight
      asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(APT + BPT) : "memory");
      floatx4 x0[TI][2], x1[TI][2];  // A of both k halves of the slab being split
      V8 ca[TI][NA], cb[TJ][NB], na[TI][NA], nb[TJ][NB];
      rdA(0, 0, x0);
      rdA(0, 1, x1);
      rdB(0, 0, cb);
      scale(x0, x1);
      sp(x0, ca);
      int kt = kt0;
      // Fast loop (K a multiple of 32 and no row of the wave scaled: every product here): no
      // branch between a k half's MFMAs and the split of the next half, which the scheduler
      // interleaves.  x0 is split before its slab's shift check and split again in the rare case
      // that the check rescales; a wave that acquires a nonzero shift finishes in the general loop.
      if (K % BK == 0 && (!S::F16 || unscaled)) {
        for (; kt < kt1; ++kt) {
          const int stg = (kt - kt0) & 1;
          rdB(stg, 1, nb);
          mm(ca, cb);
          sp_fast(x1, na);
          asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
          issue_full(min(kt + 2, kt1 - 1), stg);
          rdA(stg ^ 1, 0, x0);
          rdA(stg ^ 1, 1, x1);
          rdB(stg ^ 1, 0, cb);
          mm(na, nb);
          sp_fast(x0, ca);
          if (scale(x0, x1)) {
            sp(x0, ca);
            if (S::F16 && !unscaled) {
              ++kt;
              break;
            }
          }
        }
      }
      for (; kt < kt1; ++kt) {
        const int stg = (kt - kt0) & 1;
        rdB(stg, 1, nb);
        mm(ca, cb);
        sp(x1, na);
        asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
        issue(min(kt + 2, kt1 - 1), stg);
        rdA(stg ^ 1, 0, x0);
        rdA(stg ^ 1, 1, x1);
        rdB(stg ^ 1, 0, cb);
        mm(na, nb);
        scale(x0, x1);
        sp(x0, ca);
      }
      asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    }
    const int next = tile + stride;
    const bool more = next < t_end;
    if constexpr (S::F16) {
      // undo the scales: C = acc * 2^(E[row] + F[col]); F follows the planes of the packed B and
      // has an entry for every column of the padded n32 tiles
      int fc[TJ];
#pragma unroll
      for (int j = 0; j < TJ; ++j) fc[j] = Fc[cn0 + cbase + j * 32 + l32];
#pragma unroll
      for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int rs = __shfl(er[i], crow(r));
#pragma unroll
          for (int j = 0; j < TJ; ++j)
            acc[i][j][r] = __builtin_amdgcn_ldexpf(acc[i][j][r], rs + fc[j]);
        }
    }
    // Epilogue: stage the accumulators through LDS in row passes (one pass in mode 16), then each
    // thread applies the epilogue to float4 column groups and writes coalesced rows.  The
    // barriers wait for LDS only; the output stores stay in flight.
    {
      const bool full = cm0 + BM <= p.M && cn0 + BN <= p.N;
      float* Ct = reinterpret_cast<float*>(smem);
      for (int r0 = 0; r0 < BM; r0 += RP) {
#pragma unroll
        for (int i = 0; i < TI; ++i) {
          const int rt = rbase + i * 32 - r0;
          if (rt < 0 || rt >= RP) continue;
#pragma unroll
          for (int j = 0; j < TJ; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r)
              Ct[(rt + crow(r)) * LDT + cbase + j * 32 + l32] = acc[i][j][r];
        }
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        if (split) {
          partial_rows(g.work + g.woff[blockIdx.z] + (int64_t)blockIdx.y * p.M * p.N, p.M, p.N,
                       Ct, LDT, RP, cm0 + r0, cn0, t, NTH);
        } else switch (p.epi) {
          case EPI_SILU:
            epilogue_rows<EPI_SILU, S::F16>(p, Ct, LDT, RP, cm0 + r0, cn0, t, NTH, vec_ok, full);
            break;
          case EPI_ACCUM:
            epilogue_rows<EPI_ACCUM, S::F16>(p, Ct, LDT, RP, cm0 + r0, cn0, t, NTH, vec_ok, full);
            break;
          case EPI_PRE_SILU:
            epilogue_rows<EPI_PRE_SILU, S::F16>(p, Ct, LDT, RP, cm0 + r0, cn0, t, NTH, vec_ok, full);
            break;
          case EPI_SILU_GRAD:
            epilogue_rows<EPI_SILU_GRAD, S::F16>(p, Ct, LDT, RP, cm0 + r0, cn0, t, NTH, vec_ok, full);
            break;
          case EPI_SIGMOID:
            epilogue_rows<EPI_SIGMOID, S::F16>(p, Ct, LDT, RP, cm0 + r0, cn0, t, NTH, vec_ok, full);
            break;
          case EPI_GATE:
            epilogue_rows<EPI_GATE, S::F16>(p, Ct, LDT, RP, cm0 + r0, cn0, t, NTH, vec_ok, full,
                                            &g.gate, g.gc0[blockIdx.z]);
            break;
          case EPI_GATE_BWD:
            epilogue_rows<EPI_GATE_BWD, S::F16>(p, Ct, LDT, RP, cm0 + r0, cn0, t, NTH, vec_ok,
                                                full, &g.gate, g.gc0[blockIdx.z]);
            break;
          default:
            epilogue_rows<EPI_STORE, S::F16>(p, Ct, LDT, RP, cm0 + r0, cn0, t, NTH, vec_ok, full);
        }
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
      }
    }
    if (!more) break;
    tile = next;
    set_tile(tile);
    if (kt1 > kt0) issue(kt0, 0);
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

// ---------------------------------------------------------------------------------------------
// Short-K mode-16 products (K <= 128; plain or SiLU epilogue): the panel kernel.
//
// The tiled kernel splits a tile's A fragments once per 128-column tile, so on short-K, wide-N
// products (the radial output layer, 61440 x 1536 x 128) every tile pays the A split, a prologue
// and an LDS-staged epilogue for a k loop of four steps.  Here a workgroup of PW waves owns a
// panel of 32 PW rows and a run of 128-column tiles.  Each wave loads its 32 rows once, takes each
// row's scale over the whole of K (E = 0 while the row max is in [2^-1, 2^15), else the max lands
// below 2^kTop, as in the tiled kernel) and keeps the two fp16 planes in registers for the whole
// run.  The packed B tiles, their column exponents and the bias reach LDS by direct copies
// (buffer_load ... lds, no register round trip; F and the bias through registers).  Each output tile is computed transposed,
// D^T = B^T A^T: the packed B fragment is the MFMA's first operand and the A planes its second, so
// accumulator elements 4g .. 4g + 3 of lane l are four consecutive columns of row l % 32; the
// epilogue stages them through LDS (16 rows at a time) and stores 128-byte row segments.
// Requires ldc < 2^22 (32-bit store offsets within a wave's 32 rows).
//
// Several workgroups share a compute unit (64-column tiles: three, 43 KB of LDS each, one B tile
// buffer), so that one's MFMAs run while another waits for its stores and its next tile: loads
// (the copies among them) and stores share one counter and are not ordered with each other, so
// the only wait that guarantees the copies have landed is vmcnt(0), which also waits out the
// tile's stores.  The next tile's copies are issued as soon as every wave is done reading the
// current one, ahead of the stores, so that their latency and the stores' overlap.
constexpr int PW = 4;            // waves per panel workgroup
constexpr int PROWS = 32 * PW;   // rows per panel
constexpr int PSTR = 36;         // row stride (floats) of a wave's 16 x 32 output staging block

typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

template <int KT, int NJ>
__global__ __launch_bounds__(64 * PW, NJ == 2 ? 3 : 2) void gemm_f16x3_panel(GemmGroup g,
                                                                             int run) {
  typedef f16x8 V8;
  constexpr int TN = 32 * NJ;  // columns per tile
  const GemmArgs& p = g.p[blockIdx.z];
  const int NT32 = g.NT32[blockIdx.z];
  const int ntile = NT32 / NJ;  // TN-column tiles of the padded packed B
  const int nrun = (ntile + run - 1) / run;
  const int npanel = (p.M + PROWS - 1) / PROWS;
  if ((int)blockIdx.x >= npanel * nrun) return;
  const int panel = (int)blockIdx.x / nrun;
  const int t0 = ((int)blockIdx.x % nrun) * run, t1 = min(ntile, t0 + run);
  constexpr int S = 2 * KT;           // 16-wide k steps
  constexpr int CCH = NJ * 128;       // 16-byte chunks of one (kt, plane) chunk: [n32 (NJ)][ks][lane]
  constexpr int TCH = 2 * KT * CCH;   // 16-byte chunks of one B tile
  constexpr int PPW = TCH / 64 / PW;  // 1 KB copies per wave per tile
  __shared__ u32x4 bs[TCH];
  __shared__ u32x4 fb[2][16 * NJ];    // per tile: the column exponents F, then the bias
  __shared__ float stage[PW * 16 * PSTR];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int planes_bytes = KT * 2 * NT32 * 2048;
  // packed B and its F: every offset fits in 31 bits (checked on the host)
  const __amdgpu_buffer_rsrc_t brs =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p.B), (short)0, 0x7ffffffe, 0x00020000);
  const bool silu = p.epi == EPI_SILU;

  // B tile nt -> LDS: 1 KB copy q = 2 NJ c + sub (chunk c = 2 kt + plane holds the tile's NJ n32
  // column blocks contiguously) lands at bs + 64 q; wave w issues copies PPW w .. PPW (w + 1) - 1.
  // F and the bias go through registers: wave 0 loads F (lanes 0 .. 8 NJ - 1) and the bias (the
  // next 8 NJ lanes)
  // in one load whose address is chosen per lane (a lane without a bias value reads F and zeroes
  // it when it writes fb): a single destination register set, so that no masked part overwrites
  // registers another part's load is still filling.
  u32x4 pfb = u32x4{0u, 0u, 0u, 0u};
  bool pz = false;
  const int* Fc = reinterpret_cast<const int*>(static_cast<const char*>(p.B) + planes_bytes);
  auto copy_tile = [&](int nt) {
#pragma unroll
    for (int i = 0; i < PPW; ++i) {
      const int q = wave * PPW + i, c = q / (2 * NJ), sub = q % (2 * NJ);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(brs, (lds_ptr)(bs + 64 * q), 16, lane * 16,
                                               c * NT32 * 2048 + nt * (NJ * 2048) + sub * 1024,
                                               0, 0);
    }
    if (wave == 0) {
      const bool isb = (lane & (8 * NJ)) != 0;
      const int n = nt * TN + 4 * (lane & (8 * NJ - 1));
      const bool bok = isb && p.bias != nullptr && n < p.N;
      const void* src = bok ? static_cast<const void*>(p.bias + n)
                            : static_cast<const void*>(Fc + n);
      pfb = *static_cast<const u32x4*>(src);
      pz = isb && !bok;
    }
  };
  auto put_fb = [&](int fbuf) {
    if (wave == 0 && lane < 16 * NJ) fb[fbuf][lane] = pz ? u32x4{0u, 0u, 0u, 0u} : pfb;
  };

  // this lane's row: A[row][16 s + 8 (lane / 32) + e], e = 0..7, is the MFMA's second operand
  const int row = panel * PROWS + wave * 32 + (lane & 31);
  const bool rok = row < p.M;
  floatx4 xa[S][2];
  {
    const float* ar = p.A + (int64_t)(rok ? row : 0) * p.lda;
#pragma unroll
    for (int st = 0; st < S; ++st)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int k = 16 * st + 8 * (lane >> 5) + 4 * h;
        xa[st][h] = (rok && k < p.K) ? *reinterpret_cast<const floatx4*>(ar + k)
                                     : floatx4{0.f, 0.f, 0.f, 0.f};
      }
  }
  copy_tile(t0);
  float mx = 0.f;
#pragma unroll
  for (int st = 0; st < S; ++st)
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      mx = max3_abs(xa[st][h][0], xa[st][h][1], mx);
      mx = max3_abs(xa[st][h][2], xa[st][h][3], mx);
    }
  mx = fmaxf(mx, __shfl_xor(mx, 32));
  const int sh =
      (mx > 0.f && !(mx >= 0.5f && mx < 32768.f)) ? __builtin_amdgcn_frexp_expf(mx) - kTop : 0;
  V8 ap[S][2];
#pragma unroll
  for (int st = 0; st < S; ++st) split8_f16<2>(xa[st][0], xa[st][1], sh, ap[st]);
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): the first tile's copies have landed
  put_fb(0);
  __syncthreads();

  const bool full_rows = (panel + 1) * PROWS <= p.M;
  const int c4 = lane & 7, r8 = lane >> 3, cl = 4 * (lane >> 5), rl = lane & 31;
  // output rows through a buffer based at the wave's first row (byte offsets below 2^31: ldc is
  // checked on the host)
  const __amdgpu_buffer_rsrc_t crs = __builtin_amdgcn_make_buffer_rsrc(
      p.C + (int64_t)(panel * PROWS + wave * 32) * p.ldc, (short)0, 0x7ffffffe, 0x00020000);
  const int ldc4 = (int)p.ldc * 4;
  float* const stg = stage + wave * 16 * PSTR;
  for (int nt = t0; nt < t1; ++nt) {
    const int fbuf = (nt - t0) & 1;
    floatx16 acc[NJ];
#pragma unroll
    for (int j = 0; j < NJ; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[j][r] = 0.f;
#pragma unroll
    for (int st = 0; st < S; ++st) {
      const int kt = st >> 1, ks = st & 1;
      // the three products of mode 16, smallest first: a1 b0, a0 b1, a0 b0
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        const V8 b0 = __builtin_bit_cast(V8, bs[(2 * kt) * CCH + j * 128 + ks * 64 + lane]);
        const V8 b1 = __builtin_bit_cast(V8, bs[(2 * kt + 1) * CCH + j * 128 + ks * 64 + lane]);
        acc[j] = mfma32(b0, ap[st][1], acc[j]);
        acc[j] = mfma32(b1, ap[st][0], acc[j]);
        acc[j] = mfma32(b0, ap[st][0], acc[j]);
      }
    }
    const bool more = nt + 1 < t1;
    __syncthreads();  // every wave is done reading B tile nt
    // C = acc * 2^(E + F[col]) + bias (element 4 q + i of acc[j] is column 32 j + 8 q + cl + i),
    // through LDS one 16 x 32 block at a time: rows 16 h .. 16 h + 15 of column block j go in by
    // rows of the MFMA layout and come back as 128-byte row segments o[j][h][i] (row
    // 16 h + r8 + 8 i, columns 32 j + 4 c4 ..), so that a store instruction writes eight whole
    // rows' lines instead of 32-byte pieces of 32 rows.  All of the tile's LDS work comes before
    // the next tile's copies are issued (the compiler would otherwise wait for those copies, and
    // every store before them, at each LDS access), and the stores after them.
    const int4* fbi = reinterpret_cast<const int4*>(fb[fbuf]);
    const floatx4* fbb = reinterpret_cast<const floatx4*>(fb[fbuf] + 8 * NJ);
    floatx4 o[NJ][2][2];
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      floatx4 v[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int4 f = fbi[(32 * j + 8 * q + cl) >> 2];
        v[q][0] = __builtin_amdgcn_ldexpf(acc[j][4 * q + 0], sh + f.x);
        v[q][1] = __builtin_amdgcn_ldexpf(acc[j][4 * q + 1], sh + f.y);
        v[q][2] = __builtin_amdgcn_ldexpf(acc[j][4 * q + 2], sh + f.z);
        v[q][3] = __builtin_amdgcn_ldexpf(acc[j][4 * q + 3], sh + f.w);
      }
      const floatx4 bv = fbb[(32 * j + 4 * c4) >> 2];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        // The staging block passes values between lanes of the wave: its LDS writes and reads
        // run in program order, but a lane that skips the (masked) write has nothing ordering
        // its read after the other lanes' writes, so code motion across the block boundaries is
        // fenced off (wave_barrier: no instruction, a scheduling barrier for the wave).
        __builtin_amdgcn_wave_barrier();
        if ((rl >> 4) == h) {
#pragma unroll
          for (int q = 0; q < 4; ++q)
            *reinterpret_cast<floatx4*>(stg + (rl & 15) * PSTR + 8 * q + cl) = v[q];
        }
        __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          o[j][h][i] = *reinterpret_cast<const floatx4*>(stg + (r8 + 8 * i) * PSTR + 4 * c4) + bv;
          if (silu) {
#pragma unroll
            for (int e = 0; e < 4; ++e) o[j][h][i][e] = tta_silu(o[j][h][i][e]);
          }
        }
      }
    }
    if (more) copy_tile(nt + 1);
    // 4 NJ buffer stores, every tile: a lane whose row is past M or whose column is past N
    // stores at an offset past the buffer's end, which the hardware drops (no branches).
    {
      int coff[NJ];
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        const int n = nt * TN + 32 * j + 4 * c4;
        coff[j] = n < p.N ? 4 * n : -1;
      }
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          const int rr = 16 * h + r8 + 8 * i;
          const bool rv = full_rows || panel * PROWS + wave * 32 + rr < p.M;
#pragma unroll
          for (int j = 0; j < NJ; ++j) {
            const int off = (rv && coff[j] >= 0) ? rr * ldc4 + coff[j] : 0x7fffffff;
            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, o[j][h][i]), crs,
                                                   off, 0, 2);
          }
        }
    }
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): the copies (and the stores) are done
    if (more) put_fb(fbuf ^ 1);
    __syncthreads();
  }
}

// The panel kernel takes a mode-16 group whose products all have one KT = ceil(K / 32) <= 4, the
// plain or SiLU epilogue, no row gathers, float4-aligned outputs and at least 128 columns.
// Tiles are kPanelNJ x 32 columns wide (2: three workgroups per compute unit, 4: two);
// runs of at most kPanelRun x 128 columns keep several workgroups per compute unit.
constexpr int kPanelRun = 6, kPanelNJ = 2;

bool panel_ok(const GemmGroup& g, int n) {
  const int kt = (g.p[0].K + 31) / 32;
  if (kt < 1 || kt > 4) return false;
  for (int i = 0; i < n; ++i) {
    const GemmArgs& p = g.p[i];
    if ((p.K + 31) / 32 != kt || p.P || !g.vec[i] || (p.epi != EPI_STORE && p.epi != EPI_SILU) ||
        p.N < BN || p.ldc >= (int64_t)1 << 22)
      return false;
  }
  return true;
}

int launch_panel(GemmGroup& g, int n, hipStream_t s) {
  constexpr int NJ = kPanelNJ, RUN = kPanelRun * 4 / NJ;
  int64_t grid = 0;
  int run = 1;
  for (int i = 0; i < n; ++i) {
    const int ntile = g.NT32[i] / NJ;
    const int nr = (ntile + RUN - 1) / RUN;
    run = std::max(run, (ntile + nr - 1) / nr);
  }
  for (int i = 0; i < n; ++i) {
    const int64_t nrun = (g.NT32[i] / NJ + run - 1) / run;
    grid = std::max(grid, (int64_t)tta_blocks(g.p[i].M, PROWS) * nrun);
  }
  if (grid > (1ll << 30)) {
    tta::set_error("tta_gemm_bf16x: grid too large");
    return tta::kBadArgument;
  }
  const dim3 gd((unsigned)grid, 1, (unsigned)n), bd(64 * PW);
  switch ((g.p[0].K + 31) / 32) {
    case 1: hipLaunchKernelGGL((gemm_f16x3_panel<1, NJ>), gd, bd, 0, s, g, run); break;
    case 2: hipLaunchKernelGGL((gemm_f16x3_panel<2, NJ>), gd, bd, 0, s, g, run); break;
    case 3: hipLaunchKernelGGL((gemm_f16x3_panel<3, NJ>), gd, bd, 0, s, g, run); break;
    default: hipLaunchKernelGGL((gemm_f16x3_panel<4, NJ>), gd, bd, 0, s, g, run); break;
  }
  TTA_CHECK_LAUNCH("tta_gemm_bf16x");
  return tta::kOk;
}

// mode 16, B side: F[n] = frexp exponent of column n's max |b| minus kTop (0 for an all-zero or
// padding column).  A block of 64 columns x 16 k-strided lanes, reduced through LDS.
__global__ __launch_bounds__(1024) void k_col_exp(const float* __restrict__ B, int K, int N,
                                                  int64_t ldb, int ncol, int* __restrict__ F) {
  __shared__ float part[16][64];
  const int c = threadIdx.x & 63, kg = threadIdx.x >> 6;
  const int n = blockIdx.x * 64 + c;
  float m = 0.f;
  if (n < N)
    for (int k = kg; k < K; k += 16) m = fmaxf(m, fabsf(B[(int64_t)k * ldb + n]));
  part[kg][c] = m;
  __syncthreads();
  if (kg == 0 && n < ncol) {
#pragma unroll
    for (int q = 1; q < 16; ++q) m = fmaxf(m, part[q][c]);
    F[n] = m > 0.f ? __builtin_amdgcn_frexp_expf(m) - kTop : 0;
  }
}

// mode 16 packing: as k_pack_b with two fp16 planes of b * 2^-F[n].
__global__ __launch_bounds__(256) void k_pack_b_f16(const float* __restrict__ B, int K, int N,
                                                    int64_t ldb, int KT, int NT32,
                                                    const int* __restrict__ F,
                                                    uint4* __restrict__ out) {
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= (int64_t)KT * NT32 * 128) return;
  const int l = (int)(gid % 64);
  const int ks = (int)((gid / 64) % 2);
  const int nt = (int)((gid / 128) % NT32);
  const int kt = (int)(gid / (128 * (int64_t)NT32));
  const int n = nt * 32 + (l & 31);
  const int sh = F[n];
  float r[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int k = kt * 32 + ks * 16 + 8 * (l >> 5) + e;
    r[e] = (k < K && n < N) ? __builtin_amdgcn_ldexpf(B[(int64_t)k * ldb + n], -sh) : 0.f;
  }
  for (int q = 0; q < 2; ++q) {
    f16x8 h;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      h[e] = (_Float16)r[e];
      r[e] -= (float)h[e];
    }
    out[((((int64_t)kt * 2 + q) * NT32 + nt) * 2 + ks) * 64 + l] = __builtin_bit_cast(uint4, h);
  }
}

// One launch for the n products of g (blockIdx.z = product); each product's blocks beyond its
// own tile count exit at once.
// Blocks per product of the persistent tile loop: two per compute unit (the kernel's occupancy),
// rounded up to whole XCD rounds of 8.
// The per-device entries are atomics: host threads calling the library at the same time may both
// fill an entry, with the same value.
int persistent_cap() {
  static std::atomic<int> cap[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
  int c = cap[dev].load(std::memory_order_relaxed);
  if (c == 0) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        cus <= 0)
      cus = 256;
    c = ((2 * cus + 7) / 8) * 8;
    cap[dev].store(c, std::memory_order_relaxed);
  }
  return c;
}

template <int WM, int MODE>
int launch_bf16x(GemmGroup& g, int n, hipStream_t s, unsigned chunks = 1) {
  int64_t grid = 0;
  g.cap = persistent_cap();
  for (int i = 0; i < n; ++i) {
    const int64_t ntiles = (int64_t)tta_blocks(g.p[i].N, BN) * tta_blocks(g.p[i].M, 64 * WM);
    if (ntiles > (1ll << 30)) {
      tta::set_error("tta_gemm_bf16x: grid too large");
      return tta::kBadArgument;
    }
    grid = std::max(grid, std::min<int64_t>(((ntiles + 7) / 8) * 8, g.cap));
  }
  hipLaunchKernelGGL((gemm_bf16x_kernel<WM, MODE>), dim3((unsigned)grid, chunks, (unsigned)n),
                     dim3(128 * WM), 0, s, g);
  TTA_CHECK_LAUNCH("tta_gemm_bf16x");
  return tta::kOk;
}

bool vec_ok_of(const GemmArgs& p) {
  auto al = [](const void* q) { return q == nullptr || (uintptr_t)q % 16 == 0; };
  return p.N % 4 == 0 && p.ldc % 4 == 0 && al(p.C) && al(p.C2) && al(p.aux) && al(p.bias) &&
         (!p.P || (al(p.P) && p.ldp % 4 == 0 && p.off1 % 4 == 0));
}

int launch_mode(GemmGroup& g, int n, int mode, hipStream_t s, unsigned chunks = 1) {
  if (chunks > 1) {  // split-K: the tiled kernel (the panel kernel takes K <= 128 only)
    switch (mode) {
      case 1: return launch_bf16x<2, 1>(g, n, s, chunks);
      case 3: return launch_bf16x<2, 3>(g, n, s, chunks);
      case 16: return launch_bf16x<2, 16>(g, n, s, chunks);
      default: return launch_bf16x<2, 6>(g, n, s, chunks);
    }
  }
  switch (mode) {
    case 1: return launch_bf16x<2, 1>(g, n, s);
    case 3: return launch_bf16x<2, 3>(g, n, s);
    case 16: return panel_ok(g, n) ? launch_panel(g, n, s) : launch_bf16x<2, 16>(g, n, s);
    default: return launch_bf16x<2, 6>(g, n, s);
  }
}

// Split-K of the tiled kernel for launches too small to fill the GPU (the linears of small
// systems): when the products have fewer than 128 tiles of 128 x 128 in all, those with K >= 256
// have their K cut into chunks of whole 32-wide slabs (at least 128 columns) aiming at about 512
// workgroups; each chunk's partial product (scales undone) goes to the workspace and
// k_splitk_reduce sums the chunks in order and applies bias and epilogue.  The decision belongs
// to the launch (a product's k sums may be ordered differently in another launch).
int64_t bf16x_splitk_tiles(const tta_gemm_problem* probs, int64_t n) {
  int64_t tiles = 0;
  for (int64_t i = 0; i < n; ++i)
    if (probs[i].M > 0 && probs[i].N > 0)
      tiles += tta_blocks(probs[i].M, 128) * tta_blocks(probs[i].N, BN);
  return tiles;
}

int64_t bf16x_splitk_chunk(int64_t K, int64_t tiles) {
  const int64_t one = std::max<int64_t>(BK, (K + BK - 1) / BK * BK);  // all slabs in one chunk
  if (K < 256 || tiles >= 128) return one;
  const int64_t chunks = std::min<int64_t>((512 + tiles - 1) / tiles, K / 128);
  if (chunks < 2) return one;
  return ((K + chunks - 1) / chunks + BK - 1) / BK * BK;
}

int planes_of(int mode) {
  return mode == 1 ? 1 : mode == 3 ? 2 : mode == 6 ? 3 : mode == 16 ? 2 : 0;
}

}  // namespace

// n32 tiles of the packed B, padded with zero columns to whole 128-column block tiles so that
// every fragment a block copies exists.
static int64_t nt32_padded(int64_t N) { return ((N + BN - 1) / BN) * (BN / 32); }

extern "C" int64_t tta_pack_b_elems(int64_t K, int64_t N, int mode) {
  const int pl = planes_of(mode);
  if (pl == 0 || K <= 0 || N <= 0) return -1;
  // mode 16 appends the int32 column exponents F (two 16-bit elements each)
  return ((K + 31) / 32) * nt32_padded(N) * 1024 * pl + (mode == 16 ? nt32_padded(N) * 64 : 0);
}

extern "C" int tta_pack_b(const float* B, int64_t K, int64_t N, int64_t ldb, int mode,
                          void* out, int64_t out_elems, hipStream_t stream) {
  const int pl = planes_of(mode);
  TTA_CHECK_ARG(pl > 0, "tta_pack_b: mode must be 1, 3, 6 or 16 (got %d)", mode);
  TTA_CHECK_ARG(K > 0 && N > 0 && K < (1 << 30) && N < (1 << 30) && ldb >= N,
                "tta_pack_b: bad sizes");
  TTA_CHECK_ARG(out_elems == tta_pack_b_elems(K, N, mode), "tta_pack_b: output has %lld bf16, "
                "expected %lld", (long long)out_elems, (long long)tta_pack_b_elems(K, N, mode));
  TTA_CHECK_ARG(B && out && ((uintptr_t)out % 16 == 0), "tta_pack_b: null or misaligned pointer");
  const int KT = (int)((K + 31) / 32), NT32 = (int)nt32_padded(N);
  if (mode == 16) {
    uint4* planes = static_cast<uint4*>(out);
    int* F = reinterpret_cast<int*>(planes + (int64_t)KT * 2 * NT32 * 128);
    hipLaunchKernelGGL(k_col_exp, dim3(tta_blocks((int64_t)NT32 * 32, 64)), dim3(1024), 0, stream,
                       B, (int)K, (int)N, ldb, NT32 * 32, F);
    TTA_CHECK_LAUNCH("tta_pack_b");
    hipLaunchKernelGGL(k_pack_b_f16, dim3(tta_blocks((int64_t)KT * NT32 * 128, 256)), dim3(256), 0,
                       stream, B, (int)K, (int)N, ldb, KT, NT32, F, planes);
    TTA_CHECK_LAUNCH("tta_pack_b");
    return tta::kOk;
  }
  hipLaunchKernelGGL(k_pack_b, dim3(tta_blocks((int64_t)KT * NT32 * 128, 256)), dim3(256), 0,
                     stream, B, (int)K, (int)N, ldb, pl, KT, NT32, static_cast<uint4*>(out));
  TTA_CHECK_LAUNCH("tta_pack_b");
  return tta::kOk;
}

// Argument checks shared by the single and grouped entry points; fills p, NT32 and vec.  Returns
// kOk with *skip set for an empty product.
static int prepare_bf16x(const float* A, const void* Bp, float* C, const float* bias, float* C2,
                         const float* aux, int64_t M, int64_t N, int64_t K, int64_t lda,
                         int64_t ldc, const float* P, int64_t ldp, const int* idx0,
                         const int* idx1, int64_t off1, int64_t n_rows_p, int epilogue,
                         GemmGroup& g, int slot, bool* skip, int gate_epi = 0) {
  *skip = false;
  TTA_CHECK_ARG(M >= 0 && N >= 0 && K >= 0, "tta_gemm_bf16x: negative size");
  TTA_CHECK_ARG(M < (int64_t)1 << 31 && N < (int64_t)1 << 30 && K < (int64_t)1 << 30,
                "tta_gemm_bf16x: size exceeds int32");
  TTA_CHECK_ARG(gate_epi ? epilogue == gate_epi : (epilogue >= 0 && epilogue <= EPI_SIGMOID),
                "tta_gemm_bf16x: bad epilogue %d", epilogue);
  TTA_CHECK_ARG(epilogue != EPI_PRE_SILU || C2, "tta_gemm_bf16x: epilogue 3 needs C2");
  TTA_CHECK_ARG(epilogue != EPI_SILU_GRAD || aux, "tta_gemm_bf16x: epilogue 4 needs aux");
  TTA_CHECK_ARG(!P || (idx0 && idx1 && n_rows_p > 0 && off1 >= 0 && ldp >= off1 + N),
                "tta_gemm_bf16x: bad row-gather table");
  if (M == 0 || N == 0) {
    *skip = true;
    return tta::kOk;
  }
  TTA_CHECK_ARG(A && Bp && C, "tta_gemm_bf16x: null pointer");
  TTA_CHECK_ARG(K % 4 == 0 && lda % 4 == 0 && (uintptr_t)A % 16 == 0,
                "tta_gemm_bf16x: A needs K, lda multiples of 4 and 16-byte alignment");
  TTA_CHECK_ARG(lda >= K && ldc >= N, "tta_gemm_bf16x: leading dimension too small");
  TTA_CHECK_ARG(lda < ((int64_t)1 << 21), "tta_gemm_bf16x: lda must be below 2^21 (32-bit "
                "offsets inside a 256-row tile)");
  TTA_CHECK_ARG((uintptr_t)Bp % 16 == 0, "tta_gemm_bf16x: packed B must be 16-byte aligned");
  TTA_CHECK_ARG(tta_pack_b_elems(K, N, 6) * 2 < ((int64_t)1 << 31),
                "tta_gemm_bf16x: packed B above 2 GB (the copies use 32-bit buffer offsets)");
  g.p[slot] = GemmArgs{A, Bp, C, bias, C2, aux, (int)M, (int)N, (int)K, lda, 0, ldc, 0, 0, 0,
                       0, epilogue, P, idx0, idx1, ldp, off1};
  g.NT32[slot] = (int)nt32_padded(N);
  g.vec[slot] = vec_ok_of(g.p[slot]) ? 1 : 0;
  return tta::kOk;
}

extern "C" int tta_gemm_bf16x(const float* A, const void* Bp, float* C, const float* bias,
                              float* C2, const float* aux, int64_t M, int64_t N, int64_t K,
                              int64_t lda, int64_t ldc, int mode, const float* P, int64_t ldp,
                              const int* idx0, const int* idx1, int64_t off1, int64_t n_rows_p,
                              int epilogue, hipStream_t stream) {
  TTA_CHECK_ARG(planes_of(mode) > 0, "tta_gemm_bf16x: mode must be 1, 3, 6 or 16 (got %d)",
                mode);
  GemmGroup g{};
  bool skip = false;
  const int rc = prepare_bf16x(A, Bp, C, bias, C2, aux, M, N, K, lda, ldc, P, ldp, idx0, idx1,
                               off1, n_rows_p, epilogue, g, 0, &skip);
  if (rc != tta::kOk || skip) return rc;
  return launch_mode(g, 1, mode, stream);
}

extern "C" int tta_gemm_bf16x_group(const tta_gemm_problem* probs, int64_t n, int mode,
                                    hipStream_t stream) {
  TTA_CHECK_ARG(planes_of(mode) > 0,
                "tta_gemm_bf16x_group: mode must be 1, 3, 6 or 16 (got %d)", mode);
  TTA_CHECK_ARG(n >= 0 && n <= kMaxGroup && (probs || n == 0),
                "tta_gemm_bf16x_group: 0..%d products", kMaxGroup);
  GemmGroup g{};
  int m = 0;
  for (int64_t i = 0; i < n; ++i) {
    const tta_gemm_problem& q = probs[i];
    TTA_CHECK_ARG(q.epilogue >= 0 && q.epilogue <= EPI_SIGMOID,
                  "tta_gemm_bf16x_group: bad epilogue");
    bool skip = false;
    const int rc = prepare_bf16x(q.A, q.B, q.C, q.bias, q.C2, q.aux, q.M, q.N, q.K, q.lda, q.ldc,
                                 nullptr, 0, nullptr, nullptr, 0, 0, (int)q.epilogue, g, m,
                                 &skip);
    if (rc != tta::kOk) return rc;
    if (!skip) ++m;
  }
  if (m == 0) return tta::kOk;
  return launch_mode(g, m, mode, stream);
}

// Workspace of tta_gemm_bf16x_group_splitk in floats: the sum over products of
// ceil(K / chunk) * M * N when some product takes more than one chunk, else 0 (nothing to gain
// over tta_gemm_bf16x_group); -1 for a bad list.
extern "C" int64_t tta_gemm_bf16x_splitk_work(const tta_gemm_problem* probs, int64_t n) {
  if (n < 0 || n > kMaxGroup || (!probs && n > 0)) return -1;
  const int64_t tiles = bf16x_splitk_tiles(probs, n);
  int64_t need = 0;
  bool split = false;
  for (int64_t i = 0; i < n; ++i) {
    const tta_gemm_problem& q = probs[i];
    if (q.M <= 0 || q.N <= 0 || q.K <= 0) continue;
    const int64_t kc = bf16x_splitk_chunk(q.K, tiles);
    const int64_t chunks = (q.K + kc - 1) / kc;
    split = split || chunks > 1;
    need += (chunks * q.M * q.N + 3) / 4 * 4;  // each product's partials 16-byte aligned
  }
  return split ? need : 0;
}

// tta_gemm_bf16x_group with the k chunks of tta_gemm_bf16x_splitk_work (no row gathers); work
// NULL: never split.  gate_epi (EPI_GATE or EPI_GATE_BWD, g.gate set by the caller): every
// product has that epilogue, with first coefficient c0[i].
static int group_splitk_impl(const tta_gemm_problem* probs, int64_t n, int mode, float* work,
                             int64_t work_floats, hipStream_t stream, GemmGroup& g, int gate_epi,
                             const int64_t* c0) {
  const bool gate = gate_epi != 0;
  const char* who = gate_epi == EPI_GATE       ? "tta_gemm_bf16x_group_gate"
                    : gate_epi == EPI_GATE_BWD ? "tta_gemm_bf16x_group_gate_bwd"
                                               : "tta_gemm_bf16x_group_splitk";
  TTA_CHECK_ARG(planes_of(mode) > 0, "%s: mode must be 1, 3, 6 or 16 (got %d)", who, mode);
  TTA_CHECK_ARG(n >= 0 && n <= kMaxGroup && (probs || n == 0), "%s: 0..%d products", who,
                kMaxGroup);
  int m = 0;
  const int64_t tiles = bf16x_splitk_tiles(probs, n);
  int64_t need = 0, max_chunks = 1, max_mn = 0;
  for (int64_t i = 0; i < n; ++i) {
    const tta_gemm_problem& q = probs[i];
    TTA_CHECK_ARG(gate ? q.epilogue == gate_epi : (q.epilogue >= 0 && q.epilogue <= EPI_SIGMOID),
                  "%s: bad epilogue %lld", who, (long long)q.epilogue);
    bool skip = false;
    const int rc = prepare_bf16x(q.A, q.B, q.C, q.bias, q.C2, q.aux, q.M, q.N, q.K, q.lda, q.ldc,
                                 nullptr, 0, nullptr, nullptr, 0, 0, (int)q.epilogue, g, m,
                                 &skip, gate_epi);
    if (rc != tta::kOk) return rc;
    if (skip) continue;
    TTA_CHECK_ARG(q.K > 0, "%s: K must be positive", who);
    if (gate) {
      TTA_CHECK_ARG(q.N % g.gate.H == 0 && c0[i] >= 0 && c0[i] + q.N / g.gate.H <= 9,
                    "%s: product %lld: N = %lld columns from coefficient %lld do not fit 9 "
                    "coefficients of H = %d", who, (long long)i, (long long)q.N,
                    (long long)c0[i], g.gate.H);
      TTA_CHECK_ARG(g.vec[m], "%s: product %lld needs 16-byte aligned C, bias and row strides",
                    who, (long long)i);
      g.gc0[m] = (int)c0[i];
    }
    // the gate entry without a workspace never splits
    const int64_t kc = (!gate || work) ? bf16x_splitk_chunk(q.K, tiles) : (q.K + BK - 1) / BK * BK;
    const int64_t chunks = (q.K + kc - 1) / kc;
    g.kch[m] = (int)kc;
    g.woff[m] = need;
    need += (chunks * q.M * q.N + 3) / 4 * 4;  // each product's partials 16-byte aligned
    max_chunks = std::max(max_chunks, chunks);
    max_mn = std::max(max_mn, q.M * q.N);
    ++m;
  }
  if (m == 0) return tta::kOk;
  if (!gate || max_chunks > 1)
    TTA_CHECK_ARG(work && work_floats >= need && (uintptr_t)work % 16 == 0,
                  "%s: work holds %lld floats (16-byte aligned), needs %lld", who,
                  (long long)work_floats, (long long)need);
  if (max_chunks == 1) return launch_mode(g, m, mode, stream);  // nothing splits: direct
  TTA_CHECK_ARG(max_chunks <= 65535, "%s: too many chunks", who);
  g.work = work;
  const int rc = launch_mode(g, m, mode, stream, (unsigned)max_chunks);
  if (rc != tta::kOk) return rc;
  const int64_t rb = std::min<int64_t>((max_mn + 255) / 256, 2048);
  hipLaunchKernelGGL(k_splitk_reduce, dim3((unsigned)rb, 1, (unsigned)m), dim3(256), 0, stream, g);
  TTA_CHECK_LAUNCH(who);
  return tta::kOk;
}

extern "C" int tta_gemm_bf16x_group_splitk(const tta_gemm_problem* probs, int64_t n, int mode,
                                           float* work, int64_t work_floats,
                                           hipStream_t stream) {
  GemmGroup g{};
  return group_splitk_impl(probs, n, mode, work, work_floats, stream, g, 0, nullptr);
}

// the gate operands shared by the forward and backward gate entries
static int gate_setup(GemmGroup& g, const char* who, const int64_t* c0, const float* sig,
                      int64_t ldg, const float* x0, int64_t ldx0, int64_t H, const int* idx8) {
  TTA_CHECK_ARG(c0 && idx8 && sig && x0, "%s: null pointer", who);
  TTA_CHECK_ARG(H > 0 && H % 4 == 0 && H < (1 << 20), "%s: H = %lld must be a positive multiple "
                "of 4", who, (long long)H);
  unsigned tab = 0;
  int tmax = 0;
  for (int c = 0; c < 8; ++c) {
    TTA_CHECK_ARG(idx8[c] >= 0 && idx8[c] < 15, "%s: bad gate index", who);
    tab |= (unsigned)idx8[c] << (4 * c);
    tmax = std::max(tmax, idx8[c]);
  }
  TTA_CHECK_ARG(ldg >= (tmax + 1) * H && ldg % 4 == 0 && ldx0 >= H && ldx0 % 4 == 0 &&
                    (uintptr_t)sig % 16 == 0 && (uintptr_t)x0 % 16 == 0,
                "%s: sig / x0 rows too short or not 16-byte aligned", who);
  g.gate = GateEpi{sig, const_cast<float*>(x0), ldg, ldx0, (int)H, tab};
  return tta::kOk;
}

extern "C" int tta_gemm_bf16x_group_gate(const tta_gemm_problem* probs, int64_t n, int mode,
                                         const int64_t* c0, const float* sig, int64_t ldg,
                                         float* x0, int64_t ldx0, int64_t H, const int* idx8,
                                         float* work, int64_t work_floats, hipStream_t stream) {
  GemmGroup g{};
  const int rc = gate_setup(g, "tta_gemm_bf16x_group_gate", c0, sig, ldg, x0, ldx0, H, idx8);
  if (rc != tta::kOk) return rc;
  return group_splitk_impl(probs, n, mode, work, work_floats, stream, g, EPI_GATE, c0);
}

extern "C" int tta_gemm_bf16x_group_gate_bwd(const tta_gemm_problem* probs, int64_t n, int mode,
                                             const int64_t* c0, const float* sig, int64_t ldg,
                                             const float* x0, int64_t ldx0, int64_t H,
                                             const int* idx8, float* work, int64_t work_floats,
                                             hipStream_t stream) {
  GemmGroup g{};
  const int rc =
      gate_setup(g, "tta_gemm_bf16x_group_gate_bwd", c0, sig, ldg, x0, ldx0, H, idx8);
  if (rc != tta::kOk) return rc;
  return group_splitk_impl(probs, n, mode, work, work_floats, stream, g, EPI_GATE_BWD, c0);
}
