/* tt_atom_hip.h -- C ABI of libttatom_hip.so, the MI355X (gfx950) kernels of the eSCN-MD (UMA)
 * edgewise hot path.
 *
 * Conventions (every entry point):
 *   - device pointers to caller-allocated buffers (the PyTorch caching allocator owns memory;
 *     nothing here allocates), int64_t sizes, fp32 data, int32 indices, row-major layouts; the
 *     few small tables an entry point reads while it builds its launch (gate degree tables,
 *     rotation patterns, per-product coefficient offsets) are host arrays, as their
 *     declarations say;
 *   - work is enqueued on `stream` (hipStream_t, passed as void*), stream-ordered, reentrant
 *     (one exception: tta_virial_noalloc shares a per-GPU device array between calls, so calls
 *     of it that overlap on one GPU race; see its declaration);
 *   - return 0 on success, non-zero on bad arguments / launch failure, with the message in
 *     tta_last_error() (thread-local).  The Python layer raises RuntimeError on non-zero,
 *     matching the reference's fail-loud validation (fused_rotate_device_operation.cpp:16-44
 *     TT_FATAL -> RuntimeError, rotation.py:97-102).
 *
 * Layouts: node features [N, 9, C] natural (l, m) order; edge-frame tensors [E, 9, W] m-primed
 * order (to_m = [0,2,6,3,7,1,5,8,4]); packed Wigner coefficients [E, 35] in the reference's
 * pack order (rotation.py:196-208).  Internal edge order is destination-sorted (stable), with
 * tgt_ptr [N+1] the destination CSR and (src_ptr [N+1], src_perm [E]) the source CSR.
 */
#ifndef TT_ATOM_HIP_H
#define TT_ATOM_HIP_H

#include <stdint.h>

#include "tt_atom_hip_types.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef void* tta_stream_t; /* hipStream_t */

const char* tta_last_error(void);
int tta_version(void);
/* Writes the device's gcnArchName; non-zero unless it is gfx950. */
int tta_check_device(char* name_out, int64_t name_len);

/* ---------------------------------------------------------------- dense contractions (MFMA)
 * C[b] = epi(A[b] @ B[b] + bias[b]); A [M,K] (lda), B [K,N] (ldb), C [M,N] (ldc), batch
 * strides sA/sB/sC/sBias.  epilogue: 0 store, 1 silu, 2 accumulate, 3 store v and silu(v) to
 * C2, 4 store v * silu'(aux), 5 sigmoid (6 / 7: the gate and its input adjoint,
 * tta_gemm_bf16x_group_gate / _gate_bwd only).
 * Replaces the ttnn.linear / ttnn.matmul calls of so2.py:106-115, 282-294 (SO(2) m-block GEMMs
 * with the [[Wa,Wb],[-Wb,Wa]] fused weight of so2.py:230-253), forces.py:23-36 (_mm transpose
 * GEMMs of the VJP), spectral.py:176-187, grid.py:64-75 and model.py:223-231 (energy head). */
int tta_gemm_f32(const float* A, const float* B, float* C, const float* bias, float* C2,
                 const float* aux, int64_t M, int64_t N, int64_t K, int64_t lda, int64_t ldb,
                 int64_t ldc, int64_t batch, int64_t sA, int64_t sB, int64_t sC, int64_t sBias,
                 int epilogue, tta_stream_t stream);

/* Split GEMM on the fp16 / bf16 matrix cores (same contractions as tta_gemm_f32, same
 * epilogues, plus the optional row-gather term of tta_gemm_f32_gather when P is non-NULL).  The
 * fp32 A operand is split on the fly into planes (round-to-nearest residuals); the constant B
 * operand is packed once by tta_pack_b.  mode 16: two fp16 planes per operand, scaled by powers
 * of two (B per column at packing, A per row along K), products a0b0 + a0b1 + a1b0 -- fp32 GEMM
 * accuracy over fp32's whole range, at half the matrix work of mode 6; mode 6: 3 x 3 bf16 planes,
 * products a0b0 + a0b1 + a1b0 + a0b2 + a2b0 + a1b1 -- fp32 GEMM accuracy; mode 3: 2 x 2 bf16
 * planes, 3 products (~2^-16 relative); mode 1: bf16 operands.  A needs K, lda multiples of 4,
 * lda < 2^21 and 16-byte alignment.
 * Replaces the same ttnn.linear / ttnn.matmul call sites as tta_gemm_f32 (the reference runs
 * them in bf16 / bf8 with fp32 accumulation: compute_kernel_config, device.py). */
int64_t tta_pack_b_elems(int64_t K, int64_t N, int mode);
int tta_pack_b(const float* B, int64_t K, int64_t N, int64_t ldb, int mode, void* out,
               int64_t out_elems, tta_stream_t stream);
int tta_gemm_bf16x(const float* A, const void* Bp, float* C, const float* bias, float* C2,
                   const float* aux, int64_t M, int64_t N, int64_t K, int64_t lda, int64_t ldc,
                   int mode, const float* P, int64_t ldp, const int* idx0, const int* idx1,
                   int64_t off1, int64_t n_rows_p, int epilogue, tta_stream_t stream);

/* Up to 8 independent products in one launch (tta_gemm_problem; row-gather terms not
 * supported): the split kernel with packed B operands, or the fp32 kernel with fp32 B.
 * The three SO(2) m-block contractions of one convolution (so2.py:106-115, 282-294, and the
 * transposed products of their VJP, forces.py:23-36), which the reference issues one by one,
 * share the edge rows and run as one launch, as do the same layer of the radial MLPs of all
 * blocks.  Same checks and results as one call per product;
 * empty products are skipped. */
int tta_gemm_bf16x_group(const tta_gemm_problem* probs, int64_t n, int mode, tta_stream_t stream);
/* tta_gemm_bf16x_group for launches too small to fill the GPU (the same call sites on small
 * systems, where the fp32 kernel would otherwise run them at its matrix rate): when the products
 * have fewer than 128 tiles of 128 x 128 in all, those with K >= 256 have their K cut into
 * chunks of whole 32-wide slabs (at least 128); each chunk's partial product goes to work and a
 * second launch sums the chunks in order and applies bias and epilogue.  No row-gather term.
 * tta_gemm_bf16x_splitk_work returns the floats work (16-byte aligned) must hold (0: nothing
 * splits; -1: bad list).  Deterministic; a product's k sums may be ordered differently than in
 * another launch. */
int64_t tta_gemm_bf16x_splitk_work(const tta_gemm_problem* probs, int64_t n);
int tta_gemm_bf16x_group_splitk(const tta_gemm_problem* probs, int64_t n, int mode, float* work,
                                int64_t work_floats, tta_stream_t stream);
/* An SO(2) convolution's coefficient products with the gate of its output applied as they are
 * written (activation.py:53-70 after so2.py:282-294): every product has epilogue 6, and product
 * i's output column j is channel j % H of SH coefficient c0[i] + j / H (N a multiple of H,
 * coefficients up to 8).  Coefficient 0: C = silu(v), and v (bias included) is stored to x0
 * (rows of stride ldx0, H wide); coefficient c > 0: C = v sig[row, idx8[c-1] H + h], sig being
 * the sigmoid of the convolution's gating columns (rows of stride ldg; an earlier launch with
 * epilogue 5).  C equals tta_gate_fwd applied to the ungated products bit for bit; C, bias,
 * sig and x0 16-byte aligned with row strides and H multiples of 4.  work / work_floats as for
 * tta_gemm_bf16x_group_splitk (size from tta_gemm_bf16x_splitk_work); work NULL: never split. */
int tta_gemm_bf16x_group_gate(const tta_gemm_problem* probs, int64_t n, int mode,
                              const int64_t* c0, const float* sig, int64_t ldg, float* x0,
                              int64_t ldx0, int64_t H, const int* idx8, float* work,
                              int64_t work_floats, tta_stream_t stream);
/* The adjoint products of that convolution's VJP (forces.py:23-36, the m-block transposes) with
 * the gate's input adjoint applied as they are written (forces.py:104-130): every product has
 * epilogue 7; coefficient 0: C = v silu'(x0), coefficient c > 0: C = v sig[row, idx8[c-1] H + h]
 * (sig, x0 as kept by the forward; read only).  The gating adjoint follows from
 * tta_gate_gating_bwd.  Same layout rules, checks and work as tta_gemm_bf16x_group_gate. */
int tta_gemm_bf16x_group_gate_bwd(const tta_gemm_problem* probs, int64_t n, int mode,
                                  const int64_t* c0, const float* sig, int64_t ldg,
                                  const float* x0, int64_t ldx0, int64_t H, const int* idx8,
                                  float* work, int64_t work_floats, tta_stream_t stream);
int tta_gemm_f32_group(const tta_gemm_problem* probs, int64_t n, tta_stream_t stream);
/* tta_gemm_f32_group for launches too small to fill the GPU (the node- and edge-level linears
 * of small systems, the same call sites).  When the products have fewer than 160 tiles of
 * 32 x 64 in all, those with K >= 256 have their K cut into chunks (multiples of 64, at least
 * 128); each chunk's partial product is written to work and a second launch sums the chunks in
 * order and applies the epilogue.  A product's k sums may be ordered differently than in a
 * launch of other products; a product of one chunk gives the bits of tta_gemm_f32.
 * tta_gemm_f32_splitk_work returns the floats work must hold (0: nothing splits, use
 * tta_gemm_f32_group; -1: bad list).  Deterministic (no atomics). */
int64_t tta_gemm_f32_splitk_work(const tta_gemm_problem* probs, int64_t n);
int tta_gemm_f32_group_splitk(const tta_gemm_problem* probs, int64_t n, float* work,
                              int64_t work_floats, tta_stream_t stream);

/* ---------------------------------------------------------------- edge-frame rotation
 * out[e, m, :] = (sum_j W[e,m,j] [x[src_e, j, :] | x[tgt_e, j, :]]) * rad[e, rb(m), :]
 * x [N,9,C], out [E,9,2C], rad [E,6,2C] or NULL.  Fuses the src/tgt gather + interleave of
 * edgewise.py:52-59, rotation.rotate -> ttnn.experimental.fused_rotate (rotation.py:211-222;
 * fused_rotate.hpp:15-23) and the radial multiply of so2.py:263-277. */
int tta_gather_rotate(const float* x, const int* src, const int* tgt, const float* coef,
                      const float* rad, float* out, int64_t N, int64_t E, int64_t C,
                      tta_stream_t stream);

/* Backward of tta_gather_rotate: g_mcat [E,9,2C] (written), g_rad [E,6,2C] (written, duplicate
 * radial blocks collapsed), g_coef [E,35] (accumulated).  Replaces rotation.rotate_bw ->
 * fused_rotate (grouped by j) + fused_rotate_gc (rotation.py:225-260; fused_rotate_gc.hpp:15-23)
 * and the radial adjoint of forces.py:164-170. */
int tta_gather_rotate_bw(const float* g_xf, const float* rad, const float* x, const int* src,
                         const int* tgt, const float* coef, float* g_rad, float* g_mcat,
                         float* g_coef, int64_t N, int64_t E, int64_t C, tta_stream_t stream);

/* tta_gather_rotate_bw (rad required) walked by destination node over the destination-sorted
 * edges (tgt_ptr [N+1]): g_rad and g_coef as there; g_mcat gets its source half [.., 0:C] only,
 * and tsum [N,9,C] = the destination half summed over each node's edges in edge order (zeros for
 * a node without edges), bit-identical to tta_node_gather_sum's destination sum; g_coef's channel
 * sum runs per half (equal to tta_gather_rotate_bw's to fp32 rounding).  C a multiple of 4 with
 * C / V <= 64 (V = 4, 2, 1 for C >= 256, >= 128, smaller): C <= 64, C = 128 or C = 256.  Same
 * reference functions as tta_gather_rotate_bw plus the destination scatter of
 * forces.py:384-412, whose [E,9,C] half it never writes. */
int tta_gather_rotate_bw_dst(const float* g_xf, const float* rad, const float* x, const int* src,
                             const int* tgt_ptr, const float* coef, float* g_rad, float* g_mcat,
                             float* g_coef, float* tsum, int64_t N, int64_t E, int64_t C,
                             tta_stream_t stream);

/* The same backward, rad required, walked from both ends of every edge so that the gather
 * adjoint [E,9,2C] is never written: tta_gather_rotate_bw_srcwalk visits each node's outgoing
 * edges (src_ptr [N+1], src_perm [E]: the source CSR) and does the source half of their channels
 * [.., 0:C], tta_gather_rotate_bw_tgtwalk each node's incoming edges (tgt_ptr) and the
 * destination half [.., C:2C]; call the source walk first, on the same stream.  Each walk reads
 * a node's own row of x once and sums its half of the node adjoint over the node's edges: the
 * source walk writes ssum [N,9,C], the destination walk out[n] = (ssum[n] + its sum) + res[n]
 * (res may be NULL).  g_rad [E,6,2C]: each walk writes its half.  The coefficient adjoint: the
 * source walk writes its channel sum to coef_half [E,35], the destination walk accumulates
 * g_coef += (coef_half + its channel sum).  g_rad and out are bit-identical to
 * tta_gather_rotate_bw_dst followed by tta_node_gather_sum_dst, g_coef equal to fp32 rounding
 * (its channel sums run across lanes in another order).  C as for tta_gather_rotate_bw_dst
 * (C <= 64, C = 128 or C = 256; other widths take tta_gather_rotate_bw).  Same reference
 * functions as tta_gather_rotate_bw_dst (rotation.py:225-260, forces.py:164-170 and the
 * scatters of forces.py:384-412). */
int tta_gather_rotate_bw_srcwalk(const float* g_xf, const float* rad, const float* x,
                                 const int* src_ptr, const int* src_perm, const float* coef,
                                 float* g_rad, float* coef_half, float* ssum, int64_t N, int64_t E,
                                 int64_t C, tta_stream_t stream);
int tta_gather_rotate_bw_tgtwalk(const float* g_xf, const float* rad, const float* x,
                                 const int* tgt_ptr, const float* coef, float* g_rad,
                                 float* g_coef, const float* coef_half, const float* ssum,
                                 const float* res, float* out, int64_t N, int64_t E, int64_t C,
                                 tta_stream_t stream);

/* Source-only variant: out[e, m, :] = sum_j W[e,m,j] x[src_e, j, :], out [E, 9, C] m-primed --
 * rotation.rotate (rotation.py:211-222) applied to source features gathered by edge (the C2
 * isolated-edgewise pipeline).  Its backward writes g_in[e] = W[e]^T g_out[e] (skipped when g_in
 * is NULL) and accumulates g_coef[e, k] += <g_out[e, m_k], x[src_e, j_k]> (rotation.py:225-260). */
int tta_gather_rotate_src(const float* x, const int* src, const float* coef, float* out, int64_t N,
                          int64_t E, int64_t C, tta_stream_t stream);
int tta_gather_rotate_src_bw(const float* g_out, const float* x, const int* src, const float* coef,
                             float* g_in, float* g_coef, int64_t N, int64_t E, int64_t C,
                             tta_stream_t stream);

/* out[n] = res[n] + sum_{e in dst segment n} contrib_e, contrib = W^T (m[e] env[e]) when
 * env_first, else ((W^T pad(m[e])) env[e]) / div.  m [E, n_in, C] with n_in 9 or 3 (the m = 0
 * block only).  Deterministic (ascending edge order, no atomics).  Replaces the inverse rotate +
 * scatter of edgewise.py:72-86 (fused_rotate + one-hot matmul / scatter.segment_sum,
 * scatter.py:62-89) and the edge-degree node init of geometry.py:268-276 / edge_degree.py:43-66. */
int tta_rotate_env_segsum(const float* m, const float* coef, const float* env,
                          const int* tgt_ptr, const float* res, float* out, int64_t N, int64_t E,
                          int64_t C, int64_t n_in, int env_first, float div, tta_stream_t stream);

/* Backward of tta_rotate_env_segsum: g_m [E, n_in, C] (written), g_coef (accumulated), g_env [E]
 * (accumulated).  Replaces forces.py:366-376 and edge_degree.py:69-93. */
int tta_rotate_env_segsum_bw(const float* g_node, const int* tgt, const float* m,
                             const float* coef, const float* env, float* g_m, float* g_coef,
                             float* g_env, int64_t N, int64_t E, int64_t C, int64_t n_in,
                             int env_first, float div, tta_stream_t stream);

/* out[n] = (sum_{src(e)=n} g_mcat[e,:,0:C] + sum_{tgt(e)=n} g_mcat[e,:,C:2C]) + res[n].
 * Replaces the deinterleave + S_src / S scatters of forces.py:384-412. */
int tta_node_gather_sum(const float* g_mcat, const int* src_ptr, const int* src_perm,
                        const int* tgt_ptr, const float* res, float* out, int64_t N, int64_t E,
                        int64_t C, tta_stream_t stream);

/* tta_node_gather_sum with the destination sums given (tsum [N,9,C] from
 * tta_gather_rotate_bw_dst): out[n] = (sum_{src(e)=n} g_mcat[e,:,0:C] + tsum[n]) + res[n]. */
int tta_node_gather_sum_dst(const float* g_mcat, const int* src_ptr, const int* src_perm,
                            const float* tsum, const float* res, float* out, int64_t N, int64_t E,
                            int64_t C, tta_stream_t stream);

/* ---------------------------------------------------------------- per-op rotation and scatter
 * For callers that drive the blocks op by op (the fused step uses the kernels above).
 * tta_rotate_pattern: out[e, r, w] = sum over q in [ptr[r], ptr[r+1]) of coef[e, k[q]] *
 * x[e, blk[q], w] -- x [E, n_in, W], coef [E, nnz], out [E, n_out, W], all contiguous; the
 * pattern (ptr [n_out + 1], k and blk [nnz]) in host memory, n_in <= 255, n_out <= 64,
 * nnz <= 512.  With the pattern grouped by output row (k = the pair's index) it is
 * rotation.rotate (rotation.py:211-222, ttnn.experimental.fused_rotate, fused_rotate.hpp:15-23);
 * grouped by input column, the input half of rotation.rotate_bw (rotation.py:225-244).
 * tta_rotate_pattern_gc: gc[e, k] = sum_w g_out[e, ii[k], w] x_in[e, jj[k], w] (ii, jj host
 * arrays), the coefficient half of rotate_bw (rotation.py:246-260, fused_rotate_gc.hpp:15-23).
 * tta_segment_sum_table: out[n, w] = sum over d < Dmax of msg[gather[n Dmax + d], w] (gather a
 * device int32 [N * Dmax]; entries outside [0, n_msg), the sentinel, add nothing): segment_sum
 * over build_gather's table (scatter.py:35-89).  Fixed summation order, no atomics. */
int tta_rotate_pattern(const float* x, const float* coef, float* out, int64_t E, int64_t n_in,
                       int64_t n_out, int64_t W, int64_t nnz, const int* ptr, const int* k,
                       const int* blk, tta_stream_t stream);
int tta_rotate_pattern_gc(const float* g_out, const float* x_in, float* gc, int64_t E,
                          int64_t n_in, int64_t n_out, int64_t W, int64_t nnz, const int* ii,
                          const int* jj, tta_stream_t stream);
int tta_segment_sum_table(const float* msg, const int* gather, float* out, int64_t n_msg,
                          int64_t N, int64_t Dmax, int64_t W, tta_stream_t stream);

/* ---------------------------------------------------------------- element / row-wise
 * Gate: y[r,0] = silu(x[r,0]); y[r,c] = x[r,c] sigmoid(gating[r, idx8[c-1]]).  x [R,9,H] rows of
 * stride ldx, gating [R, L*H] rows of stride ldg (column blocks of one GEMM output allowed),
 * y / g_y contiguous [R,9,H]; g_x / g_gating share the strides of x / gating.  idx8: 8 ints in
 * host memory (read while the launch is built; likewise for tta_gate_gating_bwd and
 * tta_gemm_bf16x_group_gate(_bwd)).
 * activation.py:29-70 (m-primed idx), spectral.py:129-144 (natural idx); backward
 * forces.py:104-130 (and ttnn.experimental.fused_gate, fused_gate.hpp:14-21). */
int tta_gate_fwd(const float* x, const float* gating, float* y, int64_t R, int64_t H, int64_t L,
                 int64_t ldx, int64_t ldg, const int* idx8, tta_stream_t stream);
int tta_gate_bwd(const float* g_y, const float* x, const float* gating, float* g_x,
                 float* g_gating, int64_t R, int64_t H, int64_t L, int64_t ldx, int64_t ldg,
                 const int* idx8, tta_stream_t stream);
/* The gating adjoint of the gate above (forces.py:104-130) once the adjoint products have applied
 * its input adjoint (tta_gemm_bf16x_group_gate_bwd wrote g_x): g_gating[t] =
 * ((1 - sig[t]) / sig[t]) sum of g_x[c] y[c] over the coefficients c > 0 of index t, which is
 * sigmoid'(gating[t]) sum g_y[c] x[c] (0 where sig underflowed to 0).  y the gated rows
 * (contiguous [R,9,H]); g_x, sig and g_gating rows of strides ldgx, ldg, ldgg. */
int tta_gate_gating_bwd(const float* g_x, const float* y, const float* sig, float* g_gating,
                        int64_t R, int64_t H, int64_t L, int64_t ldgx, int64_t ldg, int64_t ldgg,
                        const int* idx8, tta_stream_t stream);

/* Radial MLP LayerNorm + SiLU: nrm = LN(a), s = silu(nrm) (so2.py:101-115) and its backward
 * g_a (so2.py:117-143; ttnn.experimental.fused_ln_bw, fused_ln_bw.hpp:14-21).  Row strides:
 * a / nrm lda, s lds, g ldg, g_a ldo.  `groups` LayerNorms of width n side by side in each row
 * (group k = columns k n .. k n + n - 1, gamma / beta [groups, n]): the radial MLPs of the
 * edge-degree embedding and of every block, which the reference runs one after another.
 * nrm may be NULL in both: the forward then does not write it and the backward recomputes it
 * from a, gamma and beta (same values as the forward's), which it then requires. */
int tta_ln_silu_fwd(const float* a, const float* gamma, const float* beta, float* nrm, float* s,
                    int64_t R, int64_t n, int64_t groups, int64_t lda, int64_t lds, float eps,
                    tta_stream_t stream);
int tta_ln_silu_bwd(const float* g, const float* a, const float* nrm, const float* gamma,
                    const float* beta, float* g_a, int64_t R, int64_t n, int64_t groups,
                    int64_t ldg, int64_t lda, int64_t ldo, float eps, tta_stream_t stream);

/* RMSNormSH (norm.py:59-111) with an optional l=0 addend (the system embedding of
 * model.py:164-167); inv [N] kept for the backward (forces.py:49-98; res = residual adjoint). */
int tta_rmsnorm_sh_fwd(const float* x, const float* aw, const float* ab, const float* add0,
                       float* y, float* inv, int64_t N, int64_t C, float eps,
                       tta_stream_t stream);
int tta_rmsnorm_sh_bwd(const float* g, const float* x, const float* aw, const float* inv,
                       const float* res, float* out, int64_t N, int64_t C, tta_stream_t stream);

int tta_silu_bwd(const float* g, const float* x, float* out, int64_t n, tta_stream_t stream);
/* Deterministic single-block sum of x[0], x[stride], ... (model.py:233-235 energy sum). */
int tta_sum(const float* x, int64_t n, int64_t stride, float* out, tta_stream_t stream);
/* out[k] = sum of x[ptr[k] .. ptr[k+1]) for k < K, each in tta_sum's order: the per-system energies
 * of a disjoint batch (model.py:241-247 energy_batch's segment sum) in one launch. */
int tta_segment_sum(const float* x, const int* ptr, int64_t K, float* out, tta_stream_t stream);
int tta_fill(float* out, int64_t n, float value, tta_stream_t stream);

/* ---------------------------------------------------------------- fused node-level stages
 * (csrc/node.hip; C and H multiples of 16 in [16, 128], lmax = 2).
 * One block's node-level tail: x2 = x1 + SpectralAtomwise(RMSNormSH_2(x1)) (model.py:158-172 with
 * norm.py:93-111 and spectral.py:146-188), saving inv2 [N], a_s [N, 2H] (pre-SiLU scalar MLP) and
 * h [N, 9, H] (pre-gate) for the backward; with awn != NULL also the next RMSNormSH of x2 (the
 * next block's norm_1 plus add0 [N, C] on coefficient 0, or the final norm with add0 = NULL)
 * into yn / invn.  ws_t [C, 2H]; w1t [3, C, H], w2t [3, H, C] per degree ([in, out]); b1 [H],
 * b2 [C] the l = 0 biases.  Replaces RMSNormSH + the spectral FF's ttnn chain + the residual add
 * + the next RMSNormSH (6 launches). */
int tta_spectral_block_fwd(const float* x1, const float* aw2, const float* ab2, const float* ws_t,
                           const float* bs, const float* w1t, const float* b1, const float* w2t,
                           const float* b2, float* inv2, float* a_s, float* h, float* x2,
                           const float* awn, const float* abn, const float* add0, float* yn,
                           float* invn, int64_t N, int64_t C, int64_t H, float eps,
                           tta_stream_t stream);
/* Its reverse (forces.py:49-98 rmsnorm_bw, 258-346 spectral_bw): g_x2 = RMSNormSH_bw(g_n; x2,
 * awn, invn) + res (res may be NULL), then g_x1 = RMSNormSH_2_bw(SpectralAtomwise_bw(g_x2)) +
 * g_x2.  w1 [3, H, C], w2 [3, C, H] per degree ([out, in]); ws [2H, C]. */
int tta_spectral_block_bwd(const float* g_n, const float* x2, const float* awn,
                           const float* invn, const float* res, const float* x1,
                           const float* aw2, const float* inv2, const float* a_s, const float* h,
                           const float* w1, const float* w2, const float* ws, float* g_x1,
                           int64_t N, int64_t C, int64_t H, tta_stream_t stream);
/* Per-node energy MLP on coefficient 0 of ne [N, 9, C] (model.py:223-231): a1 = ne0 w0t + b0,
 * a2 = silu(a1) w1t + b1, node_e = silu(a2) . w2 + b2 (w2 [H]); a1 / a2 [N, H] saved. */
int tta_energy_head_fwd(const float* ne, const float* w0t, const float* b0, const float* w1t,
                        const float* b1, const float* w2, const float* b2, float* a1, float* a2,
                        float* node_e, int64_t N, int64_t C, int64_t H, tta_stream_t stream);
/* Its adjoint for dE/dnode_e = 1 (forces.py:438-461): g_ne [N, 9, C] (coefficients 1..8 zero);
 * w0 [H, C], w1 [H, H] ([out, in]). */
int tta_energy_head_bwd(const float* a1, const float* a2, const float* w0, const float* w1,
                        const float* w2, float* g_ne, int64_t N, int64_t C, int64_t H,
                        tta_stream_t stream);

/* ---------------------------------------------------------------- geometry
 * ev = pos[src] - pos[tgt] (+ shift), dist = |ev|, coef = packed Wigner-D (geometry.py:209-224
 * + 234-240, gauge gamma; jd = [Jd_0 | Jd_1 | Jd_2] 35 floats). */
int tta_edge_wigner(const float* pos, const int* src, const int* tgt, const float* shift,
                    const float* jd, float gamma, float* ev, float* dist, float* coef, int64_t N,
                    int64_t E, tta_stream_t stream);
/* x_edge = [gaussians(dist) | src_emb[zsrc] | tgt_emb[ztgt]], env = polynomial envelope
 * (geometry.py:242-251). */
int tta_edge_features(const float* dist, const int* zsrc, const int* ztgt, const float* src_emb,
                      const float* tgt_emb, const float* offsets, float coeff, float cutoff,
                      int64_t nb, int64_t ec, float* x_edge, float* env, int64_t E,
                      tta_stream_t stream);
/* tta_edge_wigner and tta_edge_features in one launch (the forward geometry of
 * geometry.py:226-251 as the step uses it: ev, dist, coef, x_edge, env from pos); same arguments
 * and results.  Rows that are not four-column aligned (nb or ec not multiples of 4, x_edge,
 * offsets or embedding tables not 16-byte aligned) run the two kernels instead. */
int tta_edge_geometry_fwd(const float* pos, const int* src, const int* tgt, const float* shift,
                          const float* jd, float gamma, const int* zsrc, const int* ztgt,
                          const float* src_emb, const float* tgt_emb, const float* offsets,
                          float coeff, float cutoff, int64_t nb, int64_t ec, float* ev,
                          float* dist, float* coef, float* x_edge, float* env, int64_t N,
                          int64_t E, tta_stream_t stream);
/* g_ev from the coefficient, envelope and gaussian adjoints: the closed form of the host
 * torch.autograd.grad finish of forces.py:580-586 (regularised acos/atan2 of geometry.py:87-109). */
int tta_edge_geometry_bwd(const float* ev, const float* dist, const float* g_coef,
                          const float* g_env, const float* g_gauss, int64_t ldg,
                          const float* offsets, float coeff, float cutoff, int64_t nb,
                          const float* jd, float gamma, float* g_ev, int64_t E,
                          tta_stream_t stream);
/* F[n] = -(sum_{src=n} g_ev - sum_{tgt=n} g_ev) (forces.py:586-589). */
int tta_node_forces(const float* g_ev, const int* src_ptr, const int* src_perm,
                    const int* tgt_ptr, float* forces, int64_t N, int64_t E, tta_stream_t stream);
/* virial[3x3] = sum_e sym(ev (x) g_ev) = dE/dstrain (forces.py:516-524); work >= 256*9 floats. */
int tta_virial(const float* ev, const float* g_ev, int64_t E, float* work, float* out,
               tta_stream_t stream);
/* tta_virial without the `work` argument: no counterpart in the reference.  For callers that
 * cannot allocate (code under HIP graph capture, tight MD loops, harnesses that forbid
 * hipMalloc): it allocates nothing and takes its 256 * 9 partial sums (9 KB) from a device array
 * of the library, one per GPU, held until the process ends.  Limit: E <= 2^31 - 1 (the same as
 * tta_virial; the scratch size does not depend on E).  Calls that overlap on one GPU share that
 * array and race; calls in stream order do not (every call rewrites all of it). */
int tta_virial_noalloc(const float* ev, const float* g_ev, int64_t E, float* out,
                       tta_stream_t stream);

/* ---------------------------------------------------------------- Orb-v3 edge MLP + scatter
 * Internal edge order is sender-sorted (stable): sender segments are [send_ptr[n], send_ptr[n+1]),
 * receiver segments go through (recv_ptr [N+1], recv_perm [E]).  Gates sig [E, 2] hold
 * (sigmoid(receive_attn), sigmoid(send_attn)); the attention weights attn_w are [w_r | w_s]
 * (2C floats) with attn_b [2]. */

/* tta_gemm_f32 plus a row-gather term before the epilogue:
 *   v += P[idx0[row], col] + P[idx1[row], off1 + col]   (P rows of stride ldp; every idx0/idx1
 * entry must lie in [0, n_rows_p)).  The first edge-MLP layer on [e | n[send] | n[recv]]
 * (orb_model.py:248-252, the concat + ttnn.linear of MLPNorm, orb_model.py:155-173) is evaluated as
 * e @ W_e + (n @ W_s)[send] + (n @ W_r)[recv] with the node products precomputed. */
int tta_gemm_f32_gather(const float* A, const float* B, float* C, const float* bias, float* C2,
                        const float* aux, int64_t M, int64_t N, int64_t K, int64_t lda,
                        int64_t ldb, int64_t ldc, const float* P, int64_t ldp, const int* idx0,
                        const int* idx1, int64_t off1, int64_t n_rows_p, int epilogue,
                        tta_stream_t stream);

/* vec = pos[recv] - pos[send] + shift (shift may be NULL); feat [E, nb*16] = cut * rbf (x) sh;
 * cut [E].  Replaces host_edge_features (orb_geometry.py:65-97) and host_cutoff
 * (orb_model.py:69-82). */
int tta_orb_edge_features(const float* pos, const int* send, const int* recv, const float* shift,
                          float r_max, int64_t nb, float* vec, float* feat, float* cut, int64_t N,
                          int64_t E, tta_stream_t stream);
/* g_vec [E,3] from g_feat [E, nb*16] and g_cut [E]; nb a power of two.  Replaces the closed-form
 * host_edge_features_vjp (orb_geometry.py:100-133) and the host torch.autograd.grad finish of
 * orb_forces.py:303 / 374; forces then come from tta_node_forces (orb_geometry.py:135-139). */
int tta_orb_edge_features_bwd(const float* vec, const float* g_feat, const float* g_cut,
                              float r_max, int64_t nb, float* g_vec, int64_t E,
                              tta_stream_t stream);

/* Row-wise RMSNorm (eps) of h [R, C] with weight w, written to u (may be NULL), plus the residual
 * x_new = x_old + u (x_old may be NULL), inv [R] kept for the backward, and optionally the next
 * layer's attention gates on x_new into sig.  Replaces RMSNorm.__call__ (orb_model.py:107-112),
 * the residual adds (orb_model.py:266) and the gate linears + sigmoid (orb_model.py:239-244). */
int tta_rms_residual(const float* h, const float* w, const float* x_old, float* u, float* x_new,
                     float* inv, const float* attn_w, const float* attn_b, float* sig, int64_t R,
                     int64_t C, float eps, tta_stream_t stream);
/* g_h = inv w g - inv^3 / C h sum(g w h)  (rmsnorm_bw, orb_forces.py:67-79). */
int tta_rms_bwd(const float* g, const float* h, const float* w, const float* inv, float* g_h,
                int64_t R, int64_t C, tta_stream_t stream);

/* node_in [N, 3C] = [nodes | sum_recv ue sig_r cut | sum_send ue sig_s cut]: the attention-
 * weighted messages and both segment sums of orb_model.py:245-259 (scatter.segment_sum,
 * scatter.py:62-89). */
int tta_orb_segsum(const float* ue, const float* sig, const float* cut, const int* send_ptr,
                   const int* recv_ptr, const int* recv_perm, const float* nodes, float* node_in,
                   int64_t N, int64_t E, int64_t C, tta_stream_t stream);
/* Edge side of attn_layer_bw (orb_forces.py:107-147): g_h2 (written), g_cut (accumulated), g_e
 * (updated in place with the attention adjoint); g_node_in [N, 3C] from the node-MLP backward. */
int tta_orb_edge_bwd(float* g_e, const float* g_node_in, const float* ue, const float* sig,
                     const float* cut, const float* h2, const float* inv, const float* wn,
                     const float* attn_w, const int* send, const int* recv, float* g_h2,
                     float* g_cut, int64_t N, int64_t E, int64_t C, tta_stream_t stream);
/* out [N, 2H] = [sum_send x | sum_recv x] for x [E, H]: the gather adjoints of orb_forces.py:131-
 * 133 moved in front of the (linear) first-layer weight product. */
int tta_orb_node_segsum2(const float* x, const int* send_ptr, const int* recv_ptr,
                         const int* recv_perm, float* out, int64_t N, int64_t E, int64_t H,
                         tta_stream_t stream);
/* Per-system mean of node rows over [ptr[k], ptr[k+1]) (EnergyHead.batch, orb_model.py:340-355)
 * and its adjoint out[n] = g[batch[n]] / count (energy_bw_batch, orb_forces.py:207-229). */
int tta_segment_mean(const float* x, const int* ptr, float* out, int64_t K, int64_t C,
                     tta_stream_t stream);
int tta_segment_mean_bwd(const float* g, const int* batch, const int* ptr, float* out, int64_t N,
                         int64_t C, tta_stream_t stream);
/* out[n, :] = x[n, :] - (mean of x over the rows [ptr[k], ptr[k+1]) of n's system k), 1 <= C <= 16:
 * the direct ForceHead's net-force removal (orb_model.py:387-388; per system as ForceHead.batch,
 * orb_model.py:401-404).  out may alias x only if it is x itself. */
int tta_segment_center(const float* x, const int* ptr, float* out, int64_t K, int64_t C,
                       tta_stream_t stream);
/* y[r, :C] += x[r, :C] (row strides ldx, ldy): the residual adjoint sums of orb_forces.py:145. */
int tta_add_rows(const float* x, int64_t ldx, float* y, int64_t ldy, int64_t R, int64_t C,
                 tta_stream_t stream);

/* ---------------------------------------------------------------------------------------------
 * Neighbour list.  Replaces the host brute force geometry.radius_graph (geometry.py:48-81) plus
 * the per-receiver max-neighbour cap, on the device and edge for edge equal to it (same indices,
 * order and image cells).  Rows: aperiodic -> sources i (columns j ascending, edge (i, j)),
 * periodic -> receivers t (columns (j, cell) lexicographic, edge (j, t, cell)).  lo / hi
 * (nullable) bound every row's candidates to its own system of a batch.  Aperiodic keep:
 * 0 < s < mid2 with s the fp32 fma-chain norm^2 and mid2 the square of the midpoint below
 * fp32(cutoff); periodic keep: min2 < d2 <= cut2 over the image shifts [n_cells, 3], or, with
 * clo / chi (nullable, both or neither: per-row [clo, chi) ranges into that table), over the row's
 * own system's shifts -- a batch of periodic systems concatenates their tables, edge_cell then
 * indexes the concatenation (every range must lie in [0, n_cells)).
 * thresholds: the k-th smallest cap key (d2, src, cell) of every receiver (err[0] = 1 when a
 * receiver has over 1024 candidates); count: kept entries per row (thresholds null = no cap);
 * write: edges at the caller's exclusive int64 row offsets (edge_cell for periodic graphs). */
int tta_radius_graph_thresholds(const float* pos, int64_t N, const int* lo, const int* hi,
                                const float* shifts, int64_t n_cells, const int* clo,
                                const int* chi, int periodic, double mid2, float cut2,
                                float min2, int k, float* thr_d2, int* thr_src, int* thr_cell,
                                int* err, tta_stream_t stream);
int tta_radius_graph_count(const float* pos, int64_t N, const int* lo, const int* hi,
                           const float* shifts, int64_t n_cells, const int* clo, const int* chi,
                           int periodic, double mid2, float cut2, float min2,
                           const float* thr_d2, const int* thr_src, const int* thr_cell,
                           int* counts, tta_stream_t stream);
int tta_radius_graph_write(const float* pos, int64_t N, const int* lo, const int* hi,
                           const float* shifts, int64_t n_cells, const int* clo, const int* chi,
                           int periodic, double mid2, float cut2, float min2,
                           const float* thr_d2, const int* thr_src,
                           const int* thr_cell, const int64_t* offsets, int64_t* edge_src,
                           int64_t* edge_tgt, int* edge_cell, tta_stream_t stream);

/* Cell-list neighbour list: the same edges, order, image cells and cap as the three passes above
 * (and so as geometry.py:48-81 plus the cap) for one system, at O(N) cost.  Image points
 * q = pos_j (+ shift_c) are binned on grid (bins of side 1 / inv_h >= cutoff plus a rounding
 * margin, spanning the atoms' bounding box plus one bin on every side); every row scans the 27
 * bins around its atom.  build: bin_start [nbins + 1] and the binned points [n_points, 4]
 * (xyz = q, w = the int32 bits of id = j or j * n_cells + c), n_points = N (aperiodic) or
 * N * n_cells (< 2^30), with tta_cell_list_workspace(nbins, n_points) ints of workspace.
 * thresholds: as tta_radius_graph_thresholds (k in [1, 1024], any number of candidates per
 * receiver); count / write: as tta_radius_graph_count / _write; write sets err[0] = 1 (caller
 * zeroes it) and skips rows with more than 2048 kept entries, which the caller then writes with
 * tta_radius_graph_write. */
int64_t tta_cell_list_workspace(int64_t n_bins, int64_t n_points);
int tta_cell_list_build(const float* pos, int64_t N, const float* shifts, int64_t n_cells,
                        int periodic, const tta_cell_grid* grid, int* bin_start, float* points,
                        int* work, tta_stream_t stream);
int tta_radius_graph_cells_thresholds(const float* pos, int64_t N, const float* shifts,
                                      int64_t n_cells, int periodic, const tta_cell_grid* grid,
                                      const int* bin_start, const float* points, double mid2,
                                      float cut2, float min2, int k, float* thr_d2, int* thr_src,
                                      int* thr_cell, tta_stream_t stream);
int tta_radius_graph_cells_count(const float* pos, int64_t N, const float* shifts,
                                 int64_t n_cells, int periodic, const tta_cell_grid* grid,
                                 const int* bin_start, const float* points, double mid2,
                                 float cut2, float min2, const float* thr_d2, const int* thr_src,
                                 const int* thr_cell, int* counts, tta_stream_t stream);
int tta_radius_graph_cells_write(const float* pos, int64_t N, const float* shifts,
                                 int64_t n_cells, int periodic, const tta_cell_grid* grid,
                                 const int* bin_start, const float* points, double mid2,
                                 float cut2, float min2, const float* thr_d2, const int* thr_src,
                                 const int* thr_cell, const int64_t* offsets, int64_t* edge_src,
                                 int64_t* edge_tgt, int* edge_cell, int* err,
                                 tta_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* TT_ATOM_HIP_H */
