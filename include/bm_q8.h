/* SPDX-License-Identifier: MPL-2.0
 *
 * bm_q8.h — MI355X additions to the Q8 operator set, beside the reference's
 * backend interface (backend.h).  They have no counterpart in the reference:
 * the reference dispatches one Q8 matvec per weight tensor
 * (reference src/baremetal/scheduler.c:747-754,949-990) and quantizes on the
 * host (reference src/baremetal/quant.c:54-71).
 *
 * Named kernels added to the backend's kernel table (bound like any other
 * kernel through backend_encode_dispatch; buffer order listed):
 *   "quantize_q8"        {src f32 [n], dst Q8 blocks [n/32], params int{n}}
 *   "quantize_q8_bf16"   {src bf16 [n], dst Q8 blocks [n/32], params int{n}}
 *   "matmul_forward_q8_vec_multi"
 *                        {params int{nprob, n_tiles[, BT]}, plan (bm_q8_mv_plan;
 *                         bm_q8_bmv_plan when BT >= 2), weight arena,
 *                         activation arena f32, output arena f32}; BT (default
 *                         1, at most 64) rows per problem, row-major with
 *                         strides C (activations) and OC (outputs)
 *   "quantize_q4"        {src f32 [n], dst Q4 blocks [n/32], params int{n}}
 *   "quantize_q4_bf16"   {src bf16 [n], dst Q4 blocks [n/32], params int{n}}
 *   "matmul_forward_q4_vec_multi"
 *                        as matmul_forward_q8_vec_multi over Q4_0 rows, plan from
 *                        bm_q4_mv_plan
 *   "matmul_forward_q8_multi"
 *                        {params int{nprob, n_tiles[, layout]}, plan, activation arena,
 *                         weight arena, output arena f32}; layout 0: f32 row-major,
 *                         1: bf16 row-major (plans from bm_q8_gemm_plan), 2: bf16 in
 *                         MFMA fragment order written by cast_f32_bf16_frag (plans from
 *                         bm_q8_gemm_plan_frag)
 *   "cast_f32_bf16"      {src f32 [n], dst bf16 [n], params int64{n}} (round to nearest even)
 *   "cast_f32_bf16_frag" {src f32 [M][lda], dst bf16, params int{M, K, lda}}: the same
 *                        rounding into fragment order: 32-row blocks rb, 64-column steps ks
 *                        (nks = ceil(K/64) per block), four fragments s of 512 values each,
 *                        value j of lane l of fragment (rb, ks, s) at
 *                        ((rb * nks + ks) * 4 + s) * 512 + 8 l + j holding
 *                        A[32 rb + l % 32][64 ks + 32 (l / 32) + 8 s + j]; rows past M and
 *                        columns past K are zero (ceil(M/32) * nks * 2048 values)
 *   "copy_buffer"        {src, dst, params int64{nbytes}}
 *   "stream_read"        {src, sink u32 [4 * workgroups], params int64{nbytes, workgroups}}
 *                        (reads src once; the HBM read ceiling)
 *   "mfma_ceiling"       {sink f32 [256 * workgroups], params int{workgroups, iters, mode}}
 *                        (bf16 32x32x16 MFMAs, workgroups x 4 waves x iters x 8 per launch;
 *                        mode 0 register operands, 1 operands read from LDS as the prefill
 *                        GEMM's 2x2 wave tile reads them; the matrix-core ceilings)
 */
#ifndef BM_Q8_H
#define BM_Q8_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Workgroups one y = W x problem of OC rows and C columns takes in a
 * matmul_forward_q8_vec_multi launch; -1 if C is not a positive multiple of 32.
 * A launch whose problems take 4096 or more such workgroups in total keeps 12
 * rows in flight per lane instead of 8 and so takes fewer (the n_tiles that
 * bm_q8_mv_plan returns is the launch's count). */
int  bm_q8_mv_tiles(int OC, int C);

/* Writes the plan table of a matmul_forward_q8_vec_multi launch over nprob
 * problems: problem i reads Q8 rows at byte offset w_off[i] of the weight
 * arena, C[i] floats at float offset x_off[i] of the activation arena, and
 * writes OC[i] floats at float offset y_off[i] of the output arena.
 * With plan == NULL only the size is computed.  Returns the table's size in
 * bytes (plan must be 8-byte aligned and hold that many), or -1; *n_tiles
 * receives the launch's workgroup count. */
long bm_q8_mv_plan(int nprob, const uint64_t* w_off, const uint64_t* x_off, const uint64_t* y_off,
                   const int* OC, const int* C, void* plan, size_t plan_bytes, int* n_tiles);

/* The same two for a matmul_forward_q8_vec_multi (or _q4_vec_multi) launch
 * with BT >= 2 rows per problem (256 output rows per workgroup, each weight
 * read once for up to 16 rows; the same tiling for Q8_0 and Q4_0): several
 * decode sequences' projections in one launch. */
int  bm_q8_bmv_tiles(int OC, int C);
long bm_q8_bmv_plan(int nprob, const uint64_t* w_off, const uint64_t* x_off, const uint64_t* y_off,
                    const int* OC, const int* C, void* plan, size_t plan_bytes, int* n_tiles);

/* The same two for a matmul_forward_q4_vec_multi launch over Q4_0 rows
 * (20-byte blocks; w_off in bytes). */
int  bm_q4_mv_tiles(int OC, int C);
long bm_q4_mv_plan(int nprob, const uint64_t* w_off, const uint64_t* x_off, const uint64_t* y_off,
                   const int* OC, const int* C, void* plan, size_t plan_bytes, int* n_tiles);

/* Workgroups of one C[M][N] = A[M][K] x W^T prefill GEMM in a
 * matmul_forward_q8_multi launch (128 x 128 output tiles); -1 if K is not a
 * positive multiple of 32. */
int  bm_q8_gemm_tiles(int M, int N, int K);

/* Plan table of a matmul_forward_q8_multi launch: problem i reads A at
 * float offset a_off[i] (row stride lda[i]) of the activation arena, Q8
 * rows at byte offset w_off[i] of the weight arena, and writes C at float
 * offset c_off[i] (row stride ldc[i]) of the output arena.  Same return
 * convention as bm_q8_mv_plan. */
long bm_q8_gemm_plan(int nprob, const uint64_t* a_off, const uint64_t* w_off, const uint64_t* c_off,
                     const int* M, const int* N, const int* K, const int* lda, const int* ldc, void* plan,
                     size_t plan_bytes, int* n_tiles);

/* The same over fragment-ordered activations (layout 2: 256 x 96 output
 * tiles): a_off[i] is the element offset of problem i's fragment block (a
 * multiple of 512) and lda[i] its K rounded up to 64. */
int  bm_q8_gemm_tiles_frag(int M, int N, int K);
long bm_q8_gemm_plan_frag(int nprob, const uint64_t* a_off, const uint64_t* w_off, const uint64_t* c_off,
                          const int* M, const int* N, const int* K, const int* lda, const int* ldc, void* plan,
                          size_t plan_bytes, int* n_tiles);

#ifdef __cplusplus
}
#endif

#endif
