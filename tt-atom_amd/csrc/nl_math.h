// Device arithmetic shared by the row-scan (neighbors.hip) and cell-list (cells.hip) radius
// graphs: the fp32 distance predicates and cap keys evaluated exactly as the host neighbour list
// evaluates them, so both device lists keep the same edges bit for bit.
// The predicates also compile as plain C++ (no HIP headers) for the host build of the CPU tests
// (tests/host_math), with the compiler's -ffp-contract=off in place of the pragma below.
#pragma once

#if defined(__HIPCC__)
#include "common.h"
#define TTA_NL_HD __device__ __forceinline__
#else
struct float3 {
  float x, y, z;
};
inline float3 make_float3(float x, float y, float z) { return float3{x, y, z}; }
#define TTA_NL_HD inline
#endif
#include "../../include/tt_atom_hip_types.h"

// Every product and sum below is rounded on its own, as on the host: no contraction into fused
// multiply-adds.  (The toolchain's __fmul_rn / __fadd_rn are plain operators compiled with
// contraction allowed, and after inlining the backend fused x*x + y*y into an fma, with a
// different operand order in different kernels.)  The operators here are written out under
// contract(off); the only fused operations are the explicit fma calls of norm2_fma.  The pragma
// holds to the end of every source that includes this header.
#pragma clang fp contract(off)

namespace tta_nl {
TTA_NL_HD float rn_add(float a, float b) { return a + b; }
TTA_NL_HD float rn_sub(float a, float b) { return a - b; }
TTA_NL_HD float rn_mul(float a, float b) { return a * b; }
}  // namespace tta_nl

namespace tta_nl {

TTA_NL_HD float3 ld3(const float* p, int i) {
  return make_float3(p[3 * i], p[3 * i + 1], p[3 * i + 2]);
}

// torch fp32 norm^2 of a - b (the value whose rounded sqrt the host compares)
TTA_NL_HD float norm2_fma(float3 a, float3 b) {
  const float x = rn_sub(a.x, b.x), y = rn_sub(a.y, b.y), z = rn_sub(a.z, b.z);
  return __builtin_fmaf(z, z, __builtin_fmaf(y, y, rn_mul(x, x)));
}

TTA_NL_HD float sum_sq(float x, float y, float z) {
  return rn_add(rn_add(rn_mul(x, x), rn_mul(y, y)), rn_mul(z, z));
}

// periodic mask quantity: pos_t - (pos_j + sh)
TTA_NL_HD float disp2(float3 pt, float3 pj, float3 sh) {
  return sum_sq(rn_sub(pt.x, rn_add(pj.x, sh.x)), rn_sub(pt.y, rn_add(pj.y, sh.y)),
                rn_sub(pt.z, rn_add(pj.z, sh.z)));
}

// cap key distance: ev = (pos_src - pos_tgt) + sh
TTA_NL_HD float cap_d2(float3 ps, float3 pt, float3 sh) {
  return sum_sq(rn_add(rn_sub(ps.x, pt.x), sh.x), rn_add(rn_sub(ps.y, pt.y), sh.y),
                rn_add(rn_sub(ps.z, pt.z), sh.z));
}

TTA_NL_HD bool key_le(float d, int a, int c, float D, int A, int C) {
  return d < D || (d == D && (a < A || (a == A && c <= C)));
}
TTA_NL_HD bool key_lt(float d, int a, int c, float D, int A, int C) {
  return d < D || (d == D && (a < A || (a == A && c < C)));
}

#if defined(__HIPCC__)
__device__ __forceinline__ int wave_excl_scan(int v, int lane, int* total) {
  int x = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int y = __shfl_up(x, o, 64);
    if (lane >= o) x += y;
  }
  *total = __shfl(x, 63, 64);
  return x - v;
}
#endif

}  // namespace tta_nl
