/* SPDX-License-Identifier: MPL-2.0
 *
 * q8_matvec.h — problem descriptors shared by the Q8 matvec kernels, their
 * launchers and the engine's fused decode launches.
 */
#ifndef BMK_Q8_MATVEC_H
#define BMK_Q8_MATVEC_H

#include <hip/hip_runtime.h>

#define MV_MAX_PROBS 8
#define MV_U 4        /* rows in flight per lane for small launches */
#define MV_U_WIDE 8   /* rows in flight per lane when the launch has work for every CU many times over */
#define MV_U_HUGE 12  /* rows in flight per lane in a matmul_forward_q8_vec_multi launch of at least */
#define MV_HUGE_MIN_TILES 4096 /* this many MV_U_WIDE tiles (a 360M token: 5888; a 135M token: about 2200) */
#define MV_U_Q4 16    /* rows in flight per lane of the multi-matrix Q4 launch (20-byte blocks) */
#ifndef BMV_WAVES
#define BMV_WAVES 4   /* waves per workgroup of the batched (BT >= 2) multi-matrix launch */
#endif
#ifndef BMV_SUBTILES
#define BMV_SUBTILES 2 /* sub-tiles of 16 rows per wave in a plan tile of that launch, run one after the other */
#endif
#define BMV_TILE_ROWS (16 * BMV_WAVES * BMV_SUBTILES) /* output rows per plan tile of that launch */
#ifndef BMV_WSTAGES
#define BMV_WSTAGES 2  /* weight register sets of that launch: loads this many steps ahead */
#endif
#ifndef BMV_CB
#define BMV_CB 16      /* K blocks per activation chunk of that launch (staged in LDS once per chunk) */
#endif
#define BMV_IDLE_TILE 0xffffffffu /* tile-map entry of a workgroup of that launch with nothing to do */

/* One y = W x (+ bias) problem; W is OC rows of nb 36-byte Q8 blocks. */
typedef struct {
    const unsigned char* w;
    const float* x;
    float* y;
    const float* bias; /* NULL: no bias */
    int OC;
    int nb;            /* C / 32 */
    int tiles;         /* row tiles (filled by the launcher) */
    int pad_;
} MvProb;

typedef struct {
    MvProb p[MV_MAX_PROBS];
    int nprob;
} MvGroup;

/* One problem of a multi-matrix launch, addressed by offsets into three
 * arenas (weights in bytes, activations and outputs in floats).  Problem p
 * owns workgroups tile0 .. tile0+tiles-1 of the launch. */
typedef struct {
    unsigned long long w_off, x_off, y_off;
    int OC, C, tile0, tiles;
} MvDesc;

#ifdef __cplusplus
extern "C" {
#endif
int mv_tiles_for(int OC, int C, int U);
int mv_launch_group(MvGroup* g, hipStream_t s);
int mv_launch_list(const MvProb* d_probs, const unsigned int* d_tile_map, int n_tiles, hipStream_t s);
int mv_launch_multi(const unsigned char* W, const float* X, float* Y, const MvDesc* d_desc,
                    const unsigned int* d_tile_map, int n_tiles, hipStream_t s);
#ifdef __cplusplus
}
#endif

#endif
