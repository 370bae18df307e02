/* SPDX-License-Identifier: MPL-2.0
 *
 * q8_gemm.h — problem descriptors for the bf16-MFMA Q8 GEMM.
 */
#ifndef BMK_Q8_GEMM_H
#define BMK_Q8_GEMM_H

#include <hip/hip_runtime.h>

#define GM_MAX_PROBS 8

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

#ifdef __cplusplus
extern "C" {
#endif
int gm_tiles_for(int M, int N);
int gm_launch_group(GmGroup* g, hipStream_t s);
#ifdef __cplusplus
}
#endif

#endif
