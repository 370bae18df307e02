/* SPDX-License-Identifier: MPL-2.0
 *
 * pf_gemm.h — the per-layer projections of the engine's prefill, one launch
 * per projection group with its consumer fused into the epilogue.
 */
#ifndef BMK_PF_GEMM_H
#define BMK_PF_GEMM_H

#include <hip/hip_runtime.h>
#include <stddef.h>

#define PFG_MAX_PROBS 3
#define PFG_TILE 64 /* C tile columns (outputs) per workgroup, and rows (tokens) at most */
#define PFG_SS_MAX 32 /* partial sums of squares per row at most (the residual width up to 2048) */

/* Epilogues */
#define PFG_STORE 0  /* C = A W^T, each problem into its own output */
#define PFG_RESID 1  /* x += A W^T (the residual stream; one problem) */
#define PFG_SWIGLU 2 /* h = bf16(silu(A Wg^T) * (A Wu^T)); problem 0 gate, 1 up */
#define PFG_QKV 3    /* q, k, v of attention heads of size 64: q and k rotated (RoPE at each row's
                      * position), q into its output, k into the K cache, v into the V cache */

/* The prefill's weight layout (pfg_repack): a matrix of N rows of K/32
 * blocks is cut into chunks of 32 rows x one 64-wide K step (two blocks per
 * row), chunk (f, s) at (f * ceil(K / 64) + s) * CHUNK bytes.  Lane l of a
 * chunk (row 32 f + l % 32, block 2 s + l / 32) has its scale at 4 l and its
 * codes at 256 + 16 l (Q8_0: bytes 0-15; bytes 16-31 at 1280 + 16 l).  Rows
 * past N and blocks past K/32 are zero. */
#define PFG_CHUNK_Q8 2304
#define PFG_CHUNK_Q4 1280

/* One weight matrix of a launch, at w_off bytes into the prefill weight
 * arena; it owns N tiles tile0 .. (filled by pfg_launch). */
typedef struct {
    unsigned long long w_off;
    float* C; /* PFG_STORE: output, row stride ldc */
    int N, ldc, tile0, pad_;
} PfgProb;

typedef struct {
    const unsigned short* A; /* bf16 activations [M][K] in MFMA fragment order (frag_index in q8_common.h),
                              * columns K .. 64 ceil(K / 64) zero */
    const unsigned char* W;  /* prefill weight arena */
    float* x;                /* PFG_RESID: [M][N], row stride p[0].ldc */
    float* kc;               /* PFG_QKV: this layer's K cache, [KV head][dim / 4][position][4] */
    float* vc;               /*   and V cache, [position][KV], for positions 0 .. M-1 */
    const float* rope;       /*   (cos, sin) of each row's position and rotary pair, [M][32][2] */
    int MS;                  /*   cache positions */
    unsigned short* h;       /* PFG_SWIGLU: bf16 [M][N] in fragment order, columns N .. 64 ceil(N / 64) zero */
    /* RMSNorm folded into the launches around it.  A launch whose A is
     * bf16(x * g) of the residual stream scales each row of its products by
     * 1 / sqrt(ss / norm_d + eps), ss the sum of the ss_tiles partial sums
     * of squares at ss_in[tile * ss_ld + row].  A PFG_RESID launch with an
     * set writes those for the next one: an = bf16(x * gn) of the updated
     * rows in fragment order and each column tile's partial sums at
     * ss_out[tile * ss_ld + row]. */
    const float* ss_in;
    float* ss_out;
    unsigned short* an;
    const float* gn;
    int ss_tiles, ss_ld, norm_d;
    float eps;
    int M, K, NT, nprob;     /* NT: N tiles of the launch, of 32 or 64 columns (a residual launch's row sums
                              * come in NT parts); grid: M tiles of 32 or 64 rows x NT workgroups */
    PfgProb p[PFG_MAX_PROBS];
} PfgArgs;

#ifdef __cplusplus
extern "C" {
#endif
/* Bytes of an N x K matrix in the prefill weight layout (qf: 0 Q8_0, 1 Q4_0). */
size_t pfg_wbytes(int N, int K, int qf);
/* src: N rows of K/32 blocks (the reference's block format) -> dst in the prefill layout. */
int pfg_repack(const unsigned char* src, unsigned char* dst, int N, int K, int qf, hipStream_t s);
/* epi: PFG_*.  Fills NT and the problems' tile0. */
int pfg_launch(PfgArgs* a, int qf, int epi, hipStream_t s);
#ifdef __cplusplus
}
#endif

#endif
