/* SPDX-License-Identifier: MPL-2.0
 *
 * q8_plan.cpp — host-side planning for the multi-matrix Q8 matvec launch
 * (matmul_forward_q8_vec_multi): how many workgroups a problem takes and
 * the plan table {MvDesc[nprob], uint32 tile_map[n_tiles]} that the kernel
 * reads.  No device calls.
 */
#include "bmk.h"
#include "q8_matvec.h"
#include "../../include/bm_q8.h"

#include <string.h>

extern "C" int bm_q8_mv_tiles(int OC, int C) {
    if (OC <= 0 || C <= 0 || C % 32) return -1;
    return mv_tiles_for(OC, C, MV_U_WIDE);
}

extern "C" long bm_q8_mv_plan(int nprob, const uint64_t* w_off, const uint64_t* x_off, const uint64_t* y_off,
                              const int* OC, const int* C, void* plan, size_t plan_bytes, int* n_tiles_out) {
    if (nprob < 0 || (nprob > 0 && (!w_off || !x_off || !y_off || !OC || !C))) return -1;
    long tiles = 0;
    for (int i = 0; i < nprob; i++) {
        int t = bm_q8_mv_tiles(OC[i], C[i]);
        if (t < 0) return -1;
        tiles += t;
    }
    if (tiles > 0x7fffffffL) return -1;
    const size_t need = (size_t)nprob * sizeof(MvDesc) + (size_t)tiles * 4;
    if (n_tiles_out) *n_tiles_out = (int)tiles;
    if (!plan) return (long)need;
    if (plan_bytes < need || ((uintptr_t)plan & 7)) return -1;
    MvDesc* d = (MvDesc*)plan;
    unsigned int* map = (unsigned int*)((char*)plan + (size_t)nprob * sizeof(MvDesc));
    int t0 = 0;
    for (int i = 0; i < nprob; i++) {
        d[i].w_off = w_off[i];
        d[i].x_off = x_off[i];
        d[i].y_off = y_off[i];
        d[i].OC = OC[i];
        d[i].C = C[i];
        d[i].tile0 = t0;
        d[i].tiles = mv_tiles_for(OC[i], C[i], MV_U_WIDE);
        for (int k = 0; k < d[i].tiles; k++) map[t0 + k] = (unsigned int)i;
        t0 += d[i].tiles;
    }
    return (long)need;
}
