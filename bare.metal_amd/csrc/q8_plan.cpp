/* SPDX-License-Identifier: MPL-2.0
 *
 * q8_plan.cpp — host-side planning for the multi-matrix Q8 matvec launch
 * (matmul_forward_q8_vec_multi): how many workgroups a problem takes and
 * the plan table {MvDesc[nprob], uint32 tile_map[n_tiles]} that the kernel
 * reads.  No device calls.
 */
#include "bmk.h"
#include "q8_matvec.h"
#include "q8_gemm.h"

#include "bm_q8.h"

#include <string.h>

static int mv_tiles_u(int OC, int C, int U) {
    if (OC <= 0 || C <= 0 || C % 32) return -1;
    return mv_tiles_for(OC, C, U);
}

extern "C" int bm_q8_mv_tiles(int OC, int C) { return mv_tiles_u(OC, C, MV_U_WIDE); }
extern "C" int bm_q4_mv_tiles(int OC, int C) { return mv_tiles_u(OC, C, MV_U_Q4); }

/* Batched (BT >= 2) multi-matrix launch: BMV_TILE_ROWS output rows per workgroup. */
extern "C" int bm_q8_bmv_tiles(int OC, int C) {
    if (OC <= 0 || C <= 0 || C % 32) return -1;
    return (OC + BMV_TILE_ROWS - 1) / BMV_TILE_ROWS;
}

static int plan_tiles(int OC, int C, int U) { return mv_tiles_u(OC, C, U); }

/* U: rows in flight per lane of the kernel the plan is for */
static long mv_plan_u(int U, int nprob, const uint64_t* w_off, const uint64_t* x_off, const uint64_t* y_off,
                      const int* OC, const int* C, void* plan, size_t plan_bytes, int* n_tiles_out) {
    if (nprob < 0 || (nprob > 0 && (!w_off || !x_off || !y_off || !OC || !C))) return -1;
    long tiles = 0;
    for (int i = 0; i < nprob; i++) {
        int t = plan_tiles(OC[i], C[i], U);
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
    for (int i = 0; i < nprob; i++) {
        d[i].w_off = w_off[i];
        d[i].x_off = x_off[i];
        d[i].y_off = y_off[i];
        d[i].OC = OC[i];
        d[i].C = C[i];
        d[i].tiles = plan_tiles(OC[i], C[i], U);
    }
    int t0 = 0;
    for (int i = 0; i < nprob; i++) {
        d[i].tile0 = t0;
        for (int k = 0; k < d[i].tiles; k++) map[t0 + k] = (unsigned int)i;
        t0 += d[i].tiles;
    }
    return (long)need;
}

extern "C" long bm_q8_mv_plan(int nprob, const uint64_t* w_off, const uint64_t* x_off, const uint64_t* y_off,
                              const int* OC, const int* C, void* plan, size_t plan_bytes, int* n_tiles_out) {
    /* a launch with work for every CU many times over keeps more rows in flight per lane */
    long wide = 0;
    for (int i = 0; i < nprob && OC && C; i++) {
        const int t = mv_tiles_u(OC[i], C[i], MV_U_WIDE);
        if (t < 0) return -1;
        wide += t;
    }
    const int U = wide >= MV_HUGE_MIN_TILES ? MV_U_HUGE : MV_U_WIDE;
    return mv_plan_u(U, nprob, w_off, x_off, y_off, OC, C, plan, plan_bytes, n_tiles_out);
}

/* The batched launch (BT >= 2): each workgroup runs one BMV_TILE_ROWS-row
 * tile of a problem over its whole K range, staging the problem's
 * activations in LDS.  MI355X dispatches workgroup b to XCD b % 8, and each
 * XCD has its own L2: a problem whose tiles ran on every XCD would have its
 * activations fetched into all eight.  So each problem goes whole to one XCD
 * (greedy, the largest first, onto the least loaded XCD by weight bytes),
 * except one larger than a 32nd of the launch (an LM head), whose tiles are
 * cut into eight runs, one per XCD.  Within an XCD's queue the tiles run
 * longest first (decreasing C, a problem's tiles together), so the launch
 * ends on its shortest workgroups.  tile_map[8 j + x] = (problem << 16) |
 * tile is the j-th entry of XCD x's queue; shorter queues are padded with
 * BMV_IDLE_TILE (the workgroup returns at once). */
#include <algorithm>
#include <vector>
#define BMV_XCDS 8
extern "C" long bm_q8_bmv_plan(int nprob, const uint64_t* w_off, const uint64_t* x_off, const uint64_t* y_off,
                               const int* OC, const int* C, void* plan, size_t plan_bytes, int* n_tiles_out) {
    if (nprob < 0 || nprob > 0xffff || (nprob > 0 && (!w_off || !x_off || !y_off || !OC || !C))) return -1;
    std::vector<int> tiles((size_t)nprob);
    double total = 0;
    for (int i = 0; i < nprob; i++) {
        tiles[i] = bm_q8_bmv_tiles(OC[i], C[i]);
        if (tiles[i] < 0 || tiles[i] > 0xffff) return -1;
        total += (double)tiles[i] * C[i];
    }
    std::vector<int> order((size_t)nprob);
    for (int i = 0; i < nprob; i++) order[i] = i;
    std::stable_sort(order.begin(), order.end(), [&](int a, int b) {
        return (double)tiles[a] * C[a] > (double)tiles[b] * C[b];
    });
    struct Ent { int p, t; };
    std::vector<Ent> q[BMV_XCDS];
    double load[BMV_XCDS] = {0};
    for (int i : order) {
        const double cost = (double)tiles[i] * C[i];
        if (cost * 32 > total && tiles[i] >= BMV_XCDS) {
            for (int x = 0; x < BMV_XCDS; x++) {
                const int t0 = (int)((long)tiles[i] * x / BMV_XCDS), t1 = (int)((long)tiles[i] * (x + 1) / BMV_XCDS);
                for (int t = t0; t < t1; t++) q[x].push_back({i, t});
                load[x] += (double)(t1 - t0) * C[i];
            }
        } else {
            int best = 0;
            for (int x = 1; x < BMV_XCDS; x++)
                if (load[x] < load[best]) best = x;
            for (int t = 0; t < tiles[i]; t++) q[best].push_back({i, t});
            load[best] += cost;
        }
    }
    size_t longest = 0;
    for (int x = 0; x < BMV_XCDS; x++) {
        std::stable_sort(q[x].begin(), q[x].end(), [&](const Ent& a, const Ent& b) { return C[a.p] > C[b.p]; });
        longest = std::max(longest, q[x].size());
    }
    const size_t slots = BMV_XCDS * longest;
    if (slots > 0x7fffffff) return -1;
    const size_t need = (size_t)nprob * sizeof(MvDesc) + slots * 4;
    if (n_tiles_out) *n_tiles_out = (int)slots;
    if (!plan) return (long)need;
    if (plan_bytes < need || ((uintptr_t)plan & 7)) return -1;
    MvDesc* d = (MvDesc*)plan;
    unsigned int* map = (unsigned int*)((char*)plan + (size_t)nprob * sizeof(MvDesc));
    for (int i = 0; i < nprob; i++) {
        d[i].w_off = w_off[i];
        d[i].x_off = x_off[i];
        d[i].y_off = y_off[i];
        d[i].OC = OC[i];
        d[i].C = C[i];
        d[i].tile0 = 0;
        d[i].tiles = tiles[i];
    }
    for (size_t j = 0; j < longest; j++)
        for (int x = 0; x < BMV_XCDS; x++)
            map[BMV_XCDS * j + x] = j < q[x].size() ? ((unsigned int)q[x][j].p << 16) | (unsigned int)q[x][j].t
                                                    : BMV_IDLE_TILE;
    return (long)need;
}

extern "C" long bm_q4_mv_plan(int nprob, const uint64_t* w_off, const uint64_t* x_off, const uint64_t* y_off,
                              const int* OC, const int* C, void* plan, size_t plan_bytes, int* n_tiles_out) {
    return mv_plan_u(MV_U_Q4, nprob, w_off, x_off, y_off, OC, C, plan, plan_bytes, n_tiles_out);
}

extern "C" int bm_q8_gemm_tiles(int M, int N, int K) {
    if (M <= 0 || N <= 0 || K <= 0 || K % 32) return -1;
    return gm_tiles_for(M, N);
}

/* The same for fragment-ordered activations (GM_FBM x GM_FBN tiles). */
extern "C" int bm_q8_gemm_tiles_frag(int M, int N, int K) {
    if (M <= 0 || N <= 0 || K <= 0 || K % 32) return -1;
    return gm_tiles_frag(M, N);
}

/* C tile geometry of a plan: rows and columns per tile */
struct GmGeo {
    int bm, bn;
    int tiles(int M, int N) const { return ((M + bm - 1) / bm) * ((N + bn - 1) / bn); }
};
static const GmGeo GEO_ROWMAJOR = {GM_BM, GM_BN}, GEO_FRAG = {GM_FBM, GM_FBN};

/* Workgroup order of a multi-GEMM launch.  MI355X dispatches workgroup b
 * to XCD b % 8, and each XCD has its own L2.  Every (problem, N tile) pair
 * is given to one XCD, round-robin, and its M tiles run back to back
 * there: the pair's weight rows (a 128-row panel of Q8 blocks) come from
 * HBM once and are reused from that XCD's L2 by the other M tiles, and each
 * XCD keeps the activation rows it touches resident.
 * tile_map[8*j + x] = (problem << 16) | tile (row-major over the problem's
 * M x N tiles), the j-th entry of XCD x's queue; queues shorter than the
 * longest are padded with GM_IDLE_TILE (the workgroup returns at once), so
 * the launch has 8 x (longest queue) workgroups. */
#define GM_XCDS 8

/* Workgroups per XCD queue: every (problem, N tile) group goes to one XCD,
 * round robin, with its M tiles consecutive. */
static long gemm_queue_len(const GmGeo& g, int nprob, const int* M, const int* N, long* per_xcd) {
    for (int x = 0; x < GM_XCDS; x++) per_xcd[x] = 0;
    long pair = 0;
    for (int i = 0; i < nprob; i++) {
        const int tm = (M[i] + g.bm - 1) / g.bm, tn = (N[i] + g.bn - 1) / g.bn;
        for (int n = 0; n < tn; n++, pair++) per_xcd[pair % GM_XCDS] += tm;
    }
    long longest = 0;
    for (int x = 0; x < GM_XCDS; x++) longest = per_xcd[x] > longest ? per_xcd[x] : longest;
    return longest;
}

/* Plan of one multi-GEMM launch: GmDesc[nprob], then the tile map. */
static long gemm_plan_impl(const GmGeo& g, int nprob, const uint64_t* a_off, const uint64_t* w_off, const uint64_t* c_off,
                           const int* M, const int* N, const int* K, const int* lda, const int* ldc, void* plan,
                           size_t plan_bytes, int* n_tiles_out) {
    if (nprob < 0 || nprob > 0xffff || (nprob > 0 && (!a_off || !w_off || !c_off || !M || !N || !K || !lda || !ldc)))
        return -1;
    for (int i = 0; i < nprob; i++) {
        if (M[i] <= 0 || N[i] <= 0 || K[i] <= 0 || K[i] % 32) return -1;
        const int t = g.tiles(M[i], N[i]);
        if (t > 0xffff || lda[i] < K[i] || ldc[i] < N[i]) return -1;
    }
    long per_xcd[GM_XCDS];
    const long slots = (long)GM_XCDS * gemm_queue_len(g, nprob, M, N, per_xcd);
    if (slots > 0x7fffffffL) return -1;
    const size_t need = (size_t)nprob * sizeof(GmDesc) + (size_t)slots * 4;
    if (n_tiles_out) *n_tiles_out = (int)slots;
    if (!plan) return (long)need;
    if (plan_bytes < need || ((uintptr_t)plan & 7)) return -1;
    GmDesc* d = (GmDesc*)plan;
    unsigned int* map = (unsigned int*)((char*)plan + (size_t)nprob * sizeof(GmDesc));
    int t0 = 0;
    for (int i = 0; i < nprob; i++) {
        d[i].a_off = a_off[i];
        d[i].w_off = w_off[i];
        d[i].c_off = c_off[i];
        d[i].M = M[i];
        d[i].N = N[i];
        d[i].K = K[i];
        d[i].lda = lda[i];
        d[i].ldc = ldc[i];
        d[i].tile0 = t0;
        d[i].tiles = g.tiles(M[i], N[i]);
        d[i].pad_ = 0;
        t0 += d[i].tiles;
    }
    for (long b = 0; b < slots; b++) map[b] = GM_IDLE_TILE;
    long fill[GM_XCDS] = {0};
    long pair = 0;
    for (int i = 0; i < nprob; i++) {
        const int tm = (M[i] + g.bm - 1) / g.bm, tn = (N[i] + g.bn - 1) / g.bn;
        for (int n = 0; n < tn; n++, pair++) {
            const int x = (int)(pair % GM_XCDS);
            for (int m = 0; m < tm; m++)
                map[(long)GM_XCDS * fill[x]++ + x] = ((unsigned int)i << 16) | (unsigned)(m * tn + n);
        }
    }
    return (long)need;
}

extern "C" long bm_q8_gemm_plan(int nprob, const uint64_t* a_off, const uint64_t* w_off, const uint64_t* c_off,
                                const int* M, const int* N, const int* K, const int* lda, const int* ldc, void* plan,
                                size_t plan_bytes, int* n_tiles_out) {
    return gemm_plan_impl(GEO_ROWMAJOR, nprob, a_off, w_off, c_off, M, N, K, lda, ldc, plan, plan_bytes, n_tiles_out);
}

/* The plan of a launch over fragment-ordered activations (layout 2): a_off[i]
 * in elements of the bf16 fragment arena (a multiple of 512), lda[i] = K[i]
 * rounded up to 64. */
extern "C" long bm_q8_gemm_plan_frag(int nprob, const uint64_t* a_off, const uint64_t* w_off, const uint64_t* c_off,
                                     const int* M, const int* N, const int* K, const int* lda, const int* ldc,
                                     void* plan, size_t plan_bytes, int* n_tiles_out) {
    return gemm_plan_impl(GEO_FRAG, nprob, a_off, w_off, c_off, M, N, K, lda, ldc, plan, plan_bytes, n_tiles_out);
}

