/* tt_atom_hip_types.h -- plain-C argument structs of the C ABI in tt_atom_hip.h (kept in their
 * own header so that the HIP sources, which define the entry points with hipStream_t, share the
 * exact layout). */
#ifndef TT_ATOM_HIP_TYPES_H
#define TT_ATOM_HIP_TYPES_H

#include <stdint.h>

/* One product C = epi(A @ B + bias) of a grouped GEMM launch.  A [M, K] (row stride lda),
 * B: the packed bf16 planes of tta_pack_b (split-bf16 kernel) or fp32 [K, N] with row stride ldb
 * (fp32 kernel), C [M, N] (row stride ldc); bias [N], C2 and aux as for the epilogues of
 * tta_gemm_f32 (NULL when unused). */
typedef struct tta_gemm_problem {
  const float* A;
  const void* B;
  float* C;
  const float* bias;
  float* C2;
  const float* aux;
  int64_t M, N, K, lda, ldb, ldc;
  int64_t epilogue;
} tta_gemm_problem;

/* Bins of a cell-list neighbour search: bin coordinate u = (x - origin) * inv_h rounded in fp32
 * per axis, dims bins per axis (x fastest in the linear bin index). */
typedef struct tta_cell_grid {
  float origin[3];
  float inv_h;
  int dims[3];
} tta_cell_grid;

#endif
