/* SPDX-License-Identifier: MPL-2.0
 *
 * q8_gemm.h — problem descriptors for the bf16-MFMA Q8 GEMM.
 */
#ifndef BMK_Q8_GEMM_H
#define BMK_Q8_GEMM_H

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#define GM_MAX_PROBS 8
#define GM_BM 128   /* C tile rows (tokens) per workgroup */
#define GM_BN 128   /* C tile columns (output features) per workgroup */
#define GM_IDLE_TILE 0xffffffffu /* tile-map entry of a workgroup with no tile */
#define GM_FBM 256  /* fragment-ordered activations (layout 2): C tile rows per workgroup */
#define GM_FBN 96   /*   and columns (576, 192 and 1536 are multiples of 96) */
#define GM_A_F32 0  /* activation layouts of matmul_forward_q8_multi: fp32 row-major */
#define GM_A_BF16 1 /*   bf16 row-major */
#define GM_A_FRAG 2 /*   bf16 in MFMA fragment order (cast_f32_bf16_frag) */

/* C[M][N] (row stride ldc) = A[M][K] (row stride lda) x W^T, W = N rows of K/32 Q8 blocks. */
typedef struct {
    const float* A;
    const unsigned char* W;
    float* C;
    int M, N, K;
    int lda, ldc;
    int tiles;
} GmProb;

typedef struct {
    GmProb p[GM_MAX_PROBS];
    int nprob;
} GmGroup;

/* One problem of a multi-GEMM launch, addressed by offsets into three arenas
 * (activations and outputs in floats, weights in bytes); it owns workgroups
 * tile0 .. tile0+tiles-1 (row-major over its M x N tiles). */
typedef struct {
    unsigned long long a_off, w_off, c_off;
    int M, N, K, lda, ldc, tile0, tiles, pad_;
} GmDesc;

#ifdef __cplusplus
extern "C" {
#endif
int gm_tiles_for(int M, int N);
/* workgroups of one problem over fragment-ordered activations (GM_FBM x GM_FBN tiles) */
int gm_tiles_frag(int M, int N);
/* dst = bf16(src), round to nearest even, n elements */
int gm_cast_bf16(const float* src, unsigned short* dst, long n, hipStream_t s);
/* src fp32 [M][lda] -> dst bf16 [M][K] in MFMA fragment order (frag_index), padding zeroed */
int gm_cast_bf16_frag(const float* src, unsigned short* dst, int M, int K, int lda, hipStream_t s);
int gm_launch_group(GmGroup* g, hipStream_t s);
int gm_launch_group_qf(GmGroup* g, int qf, hipStream_t s);
int gm_launch_multi_qf(const void* A, int a_bf16, int qf, const unsigned char* W, float* C, const void* plan,
                       int nprob, int n_tiles, hipStream_t s);
#ifdef __cplusplus
}
#endif

#endif
