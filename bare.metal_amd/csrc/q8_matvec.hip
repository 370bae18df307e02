/* SPDX-License-Identifier: MPL-2.0
 *
 * q8_matvec.hip — decode-time Q8_0 dequant matrix-vector products on gfx950.
 *
 *   y[r] = sum_b scale[r,b] * sum_{j<32} q[r,b,j] * x[32b+j]   (+ bias[r])
 *
 * Reference semantics: matmul_forward_q8_vec (src/kernels/forward.metal:575-623)
 * for BT == 1 and matmul_forward_q8 (forward.metal:625-649) for BT > 1, with
 * the buffer order {inp, weight, bias, out, params{BT,C,OC,has_bias}}
 * (reference scheduler.c:794-799,840-847).  The weights stay in the
 * reference's array-of-structs layout: row r is C/32 consecutive 36-byte
 * blocks {f32 scale; int8 q[32]} (reference quant.h:17-32).
 *
 * gfx950 mapping (one workgroup = 256 lanes = 4 waves):
 *   - lane t owns block column b = t % nb of row slot t / nb, with
 *     nb = C/32 <= 256, so 256/nb rows are in flight per pass and every
 *     lane keeps the 32 activations of its column in registers for all rows;
 *   - a lane reads its 36-byte block with one dwordx4 + dwordx4 + dword load;
 *     consecutive lanes read consecutive blocks, so a wave streams ~2.3 KB of
 *     contiguous weight bytes per row pass;
 *   - U passes are issued before any arithmetic (U*36 bytes in flight per
 *     lane) to cover HBM latency;
 *   - the nb per-block partials of a row meet in LDS and one lane per row
 *     adds them in block order (deterministic, no atomics).
 * Rows are split into tiles of (256/nb)*U rows; a launch may cover up to
 * MV_MAX_PROBS independent problems (used to fuse q/k/v and gate/up), or an
 * arbitrary list of problems described in device memory.
 * HBM roofline: 1.125 bytes per weight + 4 bytes per x and y element.
 */
#include "bmk.h"
#include "q8_matvec.h"
#include "decode_state.h"
#include "q8_common.h"

#include <string.h>

namespace {

using namespace bmk;
constexpr int MV_THREADS = 256;

/* One row tile of one problem.  Requires nb <= MV_THREADS.  QF: block
 * format (Q8_0 36-byte or Q4_0 20-byte blocks). */
template <int U, int QF>
__device__ __forceinline__ void mv_tile(const MvProb& p, int tile, float* red) {
    typedef QFmt<QF> F;
    const int nb = p.nb;
    const int slots = MV_THREADS / nb;
    const int rows_per_tile = slots * U;
    const int t = threadIdx.x;
    const int slot = t / nb;
    const int b = t - slot * nb;
    const bool lane_on = slot < slots;
    const long row0 = (long)tile * rows_per_tile;
    const size_t row_bytes = (size_t)nb * F::BYTES;

    float xs[32];
    if (lane_on) {
        const float* xp = p.x + 32 * b;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            float4 v;
            __builtin_memcpy(&v, __builtin_assume_aligned(xp + 4 * i, 4), 16);
            xs[4 * i + 0] = v.x; xs[4 * i + 1] = v.y; xs[4 * i + 2] = v.z; xs[4 * i + 3] = v.w;
        }
    } else {
#pragma unroll
        for (int i = 0; i < 32; i++) xs[i] = 0.0f;
    }

    typename F::Block blk[U];
#pragma unroll
    for (int u = 0; u < U; u++) {
        const long r = row0 + slot + (long)u * slots;
        if (lane_on && r < p.OC) {
            blk[u] = F::load(p.w + (size_t)r * row_bytes + (size_t)b * F::BYTES);
        } else {
            blk[u] = F::zero();
        }
    }
#pragma unroll
    for (int u = 0; u < U; u++) {
        if (lane_on) red[(slot + u * slots) * nb + b] = block_dot(blk[u], xs);
    }
    __syncthreads();
    for (int rl = t; rl < rows_per_tile; rl += MV_THREADS) {
        const long r = row0 + rl;
        if (r < p.OC) {
            const float* rp = red + rl * nb;
            float acc = 0.0f;
            for (int k = 0; k < nb; k++) acc += rp[k];
            if (p.bias) acc += p.bias[r];
            p.y[r] = acc;
        }
    }
}

/* Rows longer than MV_THREADS blocks: the workgroup walks one row at a time. */
template <int QF>
__device__ __forceinline__ void mv_row_wide(const MvProb& p, long r, float* red) {
    typedef QFmt<QF> F;
    const int t = threadIdx.x;
    const unsigned char* wr = p.w + (size_t)r * p.nb * F::BYTES;
    float acc = 0.0f;
    for (int b = t; b < p.nb; b += MV_THREADS) {
        float xs[32];
        const float* xp = p.x + 32 * b;
#pragma unroll
        for (int i = 0; i < 32; i++) xs[i] = xp[i];
        acc += block_dot(F::load(wr + (size_t)b * F::BYTES), xs);
    }
    red[t] = acc;
    __syncthreads();
    if (t == 0) {
        float s = 0.0f;
        for (int k = 0; k < MV_THREADS; k++) s += red[k];
        if (p.bias) s += p.bias[r];
        p.y[r] = s;
    }
    __syncthreads();
}

template <int U, int QF>
__device__ __forceinline__ void mv_dispatch(const MvProb& p, int tile, float* red) {
    if (p.nb <= MV_THREADS) {
        mv_tile<U, QF>(p, tile, red);
    } else {
        mv_row_wide<QF>(p, tile, red);
    }
}

/* Up to MV_MAX_PROBS problems passed by value. */
template <int U>
__global__ __launch_bounds__(MV_THREADS) void k_q8_matvec(MvGroup g) {
    __shared__ float red[MV_THREADS * U];
    int tile = blockIdx.x;
    int i = 0;
    while (i + 1 < g.nprob && tile >= g.p[i].tiles) {
        tile -= g.p[i].tiles;
        i++;
    }
    mv_dispatch<U, QF_Q8>(g.p[i], tile, red);
}

/* The same over Q4_0 blocks (reference forward.metal:654-858). */
template <int U>
__global__ __launch_bounds__(MV_THREADS) void k_q4_matvec(MvGroup g) {
    __shared__ float red[MV_THREADS * U];
    int tile = blockIdx.x;
    int i = 0;
    while (i + 1 < g.nprob && tile >= g.p[i].tiles) {
        tile -= g.p[i].tiles;
        i++;
    }
    mv_dispatch<U, QF_Q4>(g.p[i], tile, red);
}

/* Any number of problems; tile_map[blockIdx.x] = (problem << 20) | tile. */
template <int U>
__global__ __launch_bounds__(MV_THREADS) void k_q8_matvec_list(const MvProb* __restrict__ probs,
                                                               const unsigned int* __restrict__ tile_map) {
    __shared__ float red[MV_THREADS * U];
    const unsigned int m = tile_map[blockIdx.x];
    const MvProb p = probs[m >> 20];
    mv_dispatch<U, QF_Q8>(p, (int)(m & 0xfffffu), red);
}

/* Any number of problems addressed by arena offsets; tile_map[blockIdx.x]
 * is the problem index, the tile is blockIdx.x - desc.tile0. */
template <int U, int QF>
__device__ __forceinline__ void mv_multi_body(const unsigned char* __restrict__ W, const float* __restrict__ X,
                                              float* __restrict__ Y, const MvDesc* __restrict__ desc,
                                              const unsigned int* __restrict__ tile_map, float* red) {
    const MvDesc d = desc[tile_map[blockIdx.x]];
    MvProb p;
    p.w = W + d.w_off;
    p.x = X + d.x_off;
    p.y = Y + d.y_off;
    p.bias = nullptr;
    p.OC = d.OC;
    p.nb = d.C / 32;
    p.tiles = d.tiles;
    p.pad_ = 0;
    mv_dispatch<U, QF>(p, (int)blockIdx.x - d.tile0, red);
}

template <int U>
__global__ __launch_bounds__(MV_THREADS) void k_q8_matvec_multi(const unsigned char* __restrict__ W,
                                                                const float* __restrict__ X, float* __restrict__ Y,
                                                                const MvDesc* __restrict__ desc,
                                                                const unsigned int* __restrict__ tile_map) {
    __shared__ float red[MV_THREADS * U];
    mv_multi_body<U, QF_Q8>(W, X, Y, desc, tile_map, red);
}

template <int U>
__global__ __launch_bounds__(MV_THREADS) void k_q4_matvec_multi(const unsigned char* __restrict__ W,
                                                                const float* __restrict__ X, float* __restrict__ Y,
                                                                const MvDesc* __restrict__ desc,
                                                                const unsigned int* __restrict__ tile_map) {
    __shared__ float red[MV_THREADS * U];
    mv_multi_body<U, QF_Q4>(W, X, Y, desc, tile_map, red);
}

/* matmul_forward_q8_vec_multi / _q4_vec_multi with BT >= 2 rows per problem
 * (several decode sequences' projections in one launch), on bf16 MFMA
 * (v_mfma_f32_16x16x32_bf16, D[16][16] += A[16][32] x B[32][16], fp32 sum).
 *
 * A workgroup is BMV_WAVES waves; it runs the BMV_TILE_ROWS-row tile
 * blockIdx.x - tile0 of problem tile_map[blockIdx.x] for batch rows
 * 16*blockIdx.y .. +15 over the whole K range, each wave 64 output rows
 * (4 groups of 16).  Per step of BMV_U K blocks:
 *   - each wave copies its 64 rows' spans of BMV_U blocks (contiguous in
 *     each row) into its own part of LDS with 16-byte loads, so every
 *     weight byte is fetched once;
 *   - the workgroup loads the step's activations once (lane t: batch row
 *     t/16, 8 consecutive columns), splits each exactly into three bf16
 *     terms (split3) and stores them in LDS in the MFMA A-operand order, so
 *     the split is paid once per 256 output rows;
 *   - per K block, lane l (c = l%16, g = l/16) reads its three A slots
 *     (x[b0 + c][32kb + 8g .. +7] as hi, mid, lo) and, per row group, the
 *     B operand q[r0 + c][32kb + 8g .. +7] (the int8 or 4-bit codes, exact
 *     in bf16) and its block scale from LDS, and chains three MFMAs.
 * Every product is exact, so each block sum is an fp32 sum of the exact
 * x * q products, as in the fp32 reference (only the order differs).  Each
 * group's block product is scaled by its row's block scale and added in
 * block order, as the reference scales each block's dot product
 * (forward.metal:575-623).  D layout: lane l holds batch rows 4*(l/16)+v of
 * output row l%16.  Problem p reads BT rows of C floats at X + x_off (row
 * stride C) and writes BT rows of OC floats at Y + y_off (row stride OC). */
typedef float bmm_f32x4 __attribute__((ext_vector_type(4)));
typedef float bmm_f32x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bmm_bf16x8 __attribute__((ext_vector_type(8)));
constexpr int BMV_GROUPS = 4; /* 16-row groups per wave */
constexpr int BMV_U = 4;      /* K blocks per step */

/* x = hi + mid + lo with three bf16 terms: hi keeps the top 8 significant
 * bits of x (truncated, so no term overflows), mid the top 8 of x - hi and
 * lo the at most 8 bits left; both subtractions are exact in fp32, so the
 * split is exact for every finite x whose lowest significant bit lies at or
 * above bf16's smallest normal (|x| >= 2^-102 suffices).  A non-finite x
 * goes whole into hi (a NaN kept a NaN) with mid = lo = 0, so its products
 * are the fp32 ones (Inf * 0 = NaN, Inf * q = Inf). */
__device__ __forceinline__ void split3(const bmm_f32x8& x, uint4& hi, uint4& mid, uint4& lo) {
    unsigned int h[8], m[8], l[8];
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const unsigned int u = __float_as_uint(x[i]);
        const bool fin = (u & 0x7f800000u) != 0x7f800000u;
        const unsigned int hb = (fin ? u : (u | ((u & 0x007fffffu) ? 0x00400000u : 0u))) & 0xffff0000u;
        const float r1 = fin ? x[i] - __uint_as_float(hb) : 0.0f;
        const unsigned int mb = __float_as_uint(r1) & 0xffff0000u;
        const float r2 = r1 - __uint_as_float(mb);
        h[i] = hb;
        m[i] = mb;
        l[i] = __float_as_uint(r2) & 0xffff0000u;
    }
    hi = make_uint4((h[0] >> 16) | h[1], (h[2] >> 16) | h[3], (h[4] >> 16) | h[5], (h[6] >> 16) | h[7]);
    mid = make_uint4((m[0] >> 16) | m[1], (m[2] >> 16) | m[3], (m[4] >> 16) | m[5], (m[6] >> 16) | m[7]);
    lo = make_uint4((l[0] >> 16) | l[1], (l[2] >> 16) | l[3], (l[4] >> 16) | l[5], (l[6] >> 16) | l[7]);
}

template <int QF>
__global__ __launch_bounds__(64 * BMV_WAVES) void k_bmv_multi(const unsigned char* __restrict__ W,
                                                              const float* __restrict__ X, float* __restrict__ Y,
                                                              const MvDesc* __restrict__ desc,
                                                              const unsigned int* __restrict__ tile_map, int BT) {
    constexpr int BYTES = QFmt<QF>::BYTES;
    constexpr int SPAN = BMV_U * BYTES;   /* bytes of one row per step: 144 (Q8_0), 80 (Q4_0) */
    constexpr int CPR = SPAN / 16;        /* 16-byte chunks per row span */
    constexpr int LDR = SPAN + 4;         /* LDS row pitch: an odd number of dwords spreads the rows over the banks */
    constexpr int LANE_OFF = QF == QF_Q4 ? 4 : 8; /* code bytes per lane and block */
    static_assert(SPAN % 16 == 0, "row span must be whole 16-byte chunks");
    static_assert(BMV_U * 32 * 16 == 64 * BMV_WAVES * 8, "one 8-column activation slot per lane and step");
    __shared__ __attribute__((aligned(16))) unsigned char tile[BMV_WAVES][64 * LDR];
    __shared__ uint4 xs[3][BMV_U][64]; /* A operands: term, block, lane */
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int c = lane & 15, g = lane >> 4;
    const MvDesc d = desc[tile_map[blockIdx.x]];
    const int row0 = ((int)blockIdx.x - d.tile0) * BMV_TILE_ROWS + 64 * wave;
    const bool wave_live = row0 < d.OC; /* the same for the whole wave */
    const int b0 = 16 * (int)blockIdx.y;
    const int nbt = min(16, BT - b0); /* batch rows of this tile */
    const int nb = d.C / 32;
    const size_t row_bytes = (size_t)nb * BYTES;
    unsigned char* wt = tile[wave];
    /* this lane's weight chunks: chunk q = lane + 64 t of the wave's 64 x CPR
     * chunk grid, row q / CPR, byte 16 (q % CPR) of the row's span; rows past
     * OC are clamped (they feed outputs never stored).  Kept as 32-bit
     * offsets from the wave's first row and LDS addresses, to spare VGPRs. */
    const unsigned char* wbase = W + d.w_off + (size_t)(wave_live ? row0 : 0) * row_bytes;
    unsigned int goff[CPR];
    int ldsa[CPR];
    int cbo[CPR]; /* the chunk's byte offset in the span, + 16 */
#pragma unroll
    for (int t = 0; t < CPR; t++) {
        const int q = lane + 64 * t, r = q / CPR, cb = 16 * (q - r * CPR);
        goff[t] = wave_live ? (unsigned int)((size_t)(min(row0 + r, d.OC - 1) - row0) * row_bytes) + cb : 0u;
        ldsa[t] = r * LDR + cb;
        cbo[t] = cb + 16;
    }
    /* this lane's activation slot: batch row xb, columns 8 * xk .. +7 of the step */
    const int xb = tid >> 4, xk = tid & 15, xu = xk >> 2, xg = xk & 3;
    const bool x_on = xb < nbt;
    const float* xr = X + d.x_off + (size_t)(b0 + (x_on ? xb : 0)) * (size_t)d.C + 8 * xk;
    /* batch rows past BT stay zero in every A slot */
    if (!x_on) {
        const uint4 z = make_uint4(0u, 0u, 0u, 0u);
        xs[0][xu][xb + 16 * xg] = z;
        xs[1][xu][xb + 16 * xg] = z;
        xs[2][xu][xb + 16 * xg] = z;
    }

    /* Loads of step kb0 into registers: the weight chunks of this wave's
     * rows (a chunk reaching past the step's bytes is moved back to end
     * there, and stored at the same place, so the overlap is written twice
     * with equal bytes: no load leaves the row) and this lane's activations. */
    /* Registers of one step's loads: the weight chunks of this wave's rows
     * (a chunk reaching past the step's bytes is moved back to end there, and
     * stored at the same place, so the overlap is written twice with equal
     * bytes: no load leaves the row) and this lane's activations.  Two sets
     * alternate, so two steps' loads are in flight while one is computed. */
    struct Stage {
        uint4 ch[CPR];
        float4 xa, xc;
        bool x_live;
    };
    Stage st0, st1;
    const int nsteps = (nb + BMV_U - 1) / BMV_U;
    /* -(bytes) a chunk moves back in a step whose row span ends `valid`
     * bytes in: 0 for a full step */
    auto chunk_shift = [&](int t, int valid) { return min(0, valid - cbo[t]); };
    /* Issues the loads of step `step` into S: every lane issues the same
     * loads whatever the step, so no branch separates two steps' loads (a
     * step past the last reads 16 bytes at the wave's first row instead, and
     * idle waves read there too); the loaded bytes of such steps are never
     * used.  Activations: a slot past the row or the batch reads the row's
     * first columns instead and is not stored. */
    auto load_step = [&](Stage& S, int step) {
        const bool real = step < nsteps;
        const int kb0 = step * BMV_U;
        S.x_live = real && x_on && kb0 + xu < nb;
        const float* xp = xr + (S.x_live ? 32 * kb0 : 0);
        __builtin_memcpy(&S.xa, __builtin_assume_aligned(xp, 16), 16);
        __builtin_memcpy(&S.xc, __builtin_assume_aligned(xp + 4, 16), 16);
        const int valid = min(BMV_U, nb - kb0) * BYTES;
        const bool wl = real && wave_live;
        const unsigned char* sb = wbase + (wl ? (size_t)kb0 * BYTES : 0);
#pragma unroll
        for (int t = 0; t < CPR; t++) {
            const int o = wl ? (int)goff[t] + chunk_shift(t, valid) : 0;
            __builtin_memcpy(&S.ch[t], __builtin_assume_aligned(sb + o, 4), 16);
        }
    };

    bmm_f32x4 acc[BMV_GROUPS];
#pragma unroll
    for (int j = 0; j < BMV_GROUPS; j++) acc[j] = bmm_f32x4{0.f, 0.f, 0.f, 0.f};

    /* One step: stage S (the loads of step `step`) into LDS, issue the loads
     * of step + 2 into S, then the step's products. */
    auto run_step = [&](Stage& S, int step) {
        const int kb0 = step * BMV_U;
        __syncthreads(); /* the previous step's LDS reads are done */
        if (wave_live) {
            const int valid = min(BMV_U, nb - kb0) * BYTES;
#pragma unroll
            for (int t = 0; t < CPR; t++) {
                const int la = ldsa[t] + chunk_shift(t, valid);
                unsigned int w4[4] = {S.ch[t].x, S.ch[t].y, S.ch[t].z, S.ch[t].w};
                /* 4-byte stores: a moved-back chunk is 4-byte but not 16-byte aligned */
#pragma unroll
                for (int e = 0; e < 4; e++) *(unsigned int*)&wt[la + 4 * e] = w4[e];
            }
        }
        if (S.x_live) {
            const bmm_f32x8 xf = {S.xa.x, S.xa.y, S.xa.z, S.xa.w, S.xc.x, S.xc.y, S.xc.z, S.xc.w};
            uint4 th, tm, tl;
            split3(xf, th, tm, tl);
            xs[0][xu][xb + 16 * xg] = th;
            xs[1][xu][xb + 16 * xg] = tm;
            xs[2][xu][xb + 16 * xg] = tl;
        }
        __syncthreads();
        /* the loads two steps ahead fly while this step's products run */
        load_step(S, step + 2);
        if (!wave_live) return;
#pragma unroll
        for (int u = 0; u < BMV_U; u++) {
            /* blocks past the row (last step only; the same for the whole
             * wave) are skipped, not weighted by 0: 0 * Inf would be NaN */
            if (kb0 + u >= nb) break;
            bmm_bf16x8 xh, xm, xl;
            {
                const uint4 a0 = xs[0][u][lane], a1 = xs[1][u][lane], a2 = xs[2][u][lane];
                __builtin_memcpy(&xh, &a0, 16);
                __builtin_memcpy(&xm, &a1, 16);
                __builtin_memcpy(&xl, &a2, 16);
            }
            bmm_bf16x8 wv[BMV_GROUPS];
            float sc[BMV_GROUPS];
#pragma unroll
            for (int j = 0; j < BMV_GROUPS; j++) {
                const unsigned char* blk = &wt[(16 * j + c) * LDR + u * BYTES];
                sc[j] = *(const float*)blk;
                const unsigned int q0 = *(const unsigned int*)(blk + 4 + LANE_OFF * g);
                const unsigned int q1 = QF == QF_Q8 ? *(const unsigned int*)(blk + 8 + LANE_OFF * g) : 0u;
                bmm_f32x8 w;
                if (QF == QF_Q4) {
#pragma unroll
                    for (int i = 0; i < 8; i++) w[i] = q4_code(q0, i);
                } else {
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        w[i] = q8_byte(q0, i);
                        w[4 + i] = q8_byte(q1, i);
                    }
                }
                wv[j] = __builtin_convertvector(w, bmm_bf16x8);
            }
            bmm_f32x4 dd[BMV_GROUPS];
#pragma unroll
            for (int j = 0; j < BMV_GROUPS; j++)
                dd[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xh, wv[j], bmm_f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
#pragma unroll
            for (int j = 0; j < BMV_GROUPS; j++) dd[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xm, wv[j], dd[j], 0, 0, 0);
#pragma unroll
            for (int j = 0; j < BMV_GROUPS; j++) dd[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xl, wv[j], dd[j], 0, 0, 0);
#pragma unroll
            for (int j = 0; j < BMV_GROUPS; j++)
#pragma unroll
                for (int v = 0; v < 4; v++) acc[j][v] = fmaf(sc[j], dd[j][v], acc[j][v]);
        }
    };

    load_step(st0, 0);
    load_step(st1, 1);
    int step = 0;
    for (; step + 1 < nsteps; step += 2) {
        run_step(st0, step);
        run_step(st1, step + 1);
    }
    if (step < nsteps) run_step(st0, step);
    if (!wave_live) return;
#pragma unroll
    for (int j = 0; j < BMV_GROUPS; j++) {
        const int row = row0 + 16 * j + c;
        if (row < d.OC) {
            float* y = Y + d.y_off + row;
#pragma unroll
            for (int v = 0; v < 4; v++) {
                const int b = b0 + 4 * g + v;
                if (b < BT) y[(size_t)b * d.OC] = acc[j][v];
            }
        }
    }
}

} // namespace

/* The batched multi-matrix launch; the caller has checked the plan against
 * the arenas. */
static int launch_bmv_multi(int qf, const unsigned char* W, const float* X, float* Y, const MvDesc* d_desc,
                            const unsigned int* d_tile_map, int n_tiles, int BT, hipStream_t s) {
    if (n_tiles <= 0 || BT < 2 || BT > DEC_MAX_B) return -1;
    const dim3 grid((unsigned)n_tiles, (unsigned)((BT + 15) / 16));
    if (qf == QF_Q4)
        hipLaunchKernelGGL(k_bmv_multi<QF_Q4>, grid, dim3(64 * BMV_WAVES), 0, s, W, X, Y, d_desc, d_tile_map, BT);
    else
        hipLaunchKernelGGL(k_bmv_multi<QF_Q8>, grid, dim3(64 * BMV_WAVES), 0, s, W, X, Y, d_desc, d_tile_map, BT);
    BMK_LAUNCH_CHECK();
    return 0;
}

/* ------------------------------------------------------------------ */

extern "C" int mv_tiles_for(int OC, int C, int U) {
    const int nb = C / 32;
    if (nb > MV_THREADS) return OC;
    const int rows = (MV_THREADS / nb) * U;
    return (OC + rows - 1) / rows;
}

/* Tiles at MV_U from which a launch uses MV_U_WIDE rows per lane: at least
 * 384 workgroups at the wider tile, 1.5 per CU of MI355X's 256.  More bytes
 * in flight per lane is what lifts a streaming matvec toward the HBM
 * roofline; fewer, wider tiles would starve the CUs on small matrices.
 * Measured on the 49152-row LM heads, launch after launch over weights no
 * cache holds: 12.9 us at 8 rows per lane against 14.1 at 4 (x960), 9.5
 * against 9.8 (x576); 1 or 2 rows per lane are slower, 16 too. */
#define MV_WIDE_MIN_TILES 768

template <int QF>
static int launch_group(MvGroup* g, hipStream_t s) {
    long total = 0;
    for (int i = 0; i < g->nprob; i++) total += mv_tiles_for(g->p[i].OC, g->p[i].nb * 32, MV_U);
    if (total <= 0) return 0;
    const int U = total >= MV_WIDE_MIN_TILES ? MV_U_WIDE : MV_U;
    total = 0;
    for (int i = 0; i < g->nprob; i++) {
        g->p[i].tiles = mv_tiles_for(g->p[i].OC, g->p[i].nb * 32, U);
        total += g->p[i].tiles;
    }
    const dim3 grid((unsigned)total), tb(MV_THREADS);
    if (QF == QF_Q4) {
        if (U == MV_U_WIDE) hipLaunchKernelGGL(k_q4_matvec<MV_U_WIDE>, grid, tb, 0, s, *g);
        else hipLaunchKernelGGL(k_q4_matvec<MV_U>, grid, tb, 0, s, *g);
    } else {
        if (U == MV_U_WIDE) hipLaunchKernelGGL(k_q8_matvec<MV_U_WIDE>, grid, tb, 0, s, *g);
        else hipLaunchKernelGGL(k_q8_matvec<MV_U>, grid, tb, 0, s, *g);
    }
    BMK_LAUNCH_CHECK();
    return 0;
}

extern "C" int mv_launch_group(MvGroup* g, hipStream_t s) { return launch_group<QF_Q8>(g, s); }

extern "C" int mv_launch_list(const MvProb* d_probs, const unsigned int* d_tile_map, int n_tiles, hipStream_t s) {
    if (n_tiles <= 0) return 0;
    hipLaunchKernelGGL(k_q8_matvec_list<MV_U>, dim3((unsigned)n_tiles), dim3(MV_THREADS), 0, s, d_probs,
                       d_tile_map);
    BMK_LAUNCH_CHECK();
    return 0;
}

template <int QF>
static int launch_multi(const unsigned char* W, const float* X, float* Y, const MvDesc* d_desc,
                        const unsigned int* d_tile_map, int n_tiles, hipStream_t s, int U = MV_U_WIDE) {
    if (n_tiles <= 0) return 0;
    if (QF == QF_Q4)
        hipLaunchKernelGGL(k_q4_matvec_multi<MV_U_Q4>, dim3((unsigned)n_tiles), dim3(MV_THREADS), 0, s, W, X, Y,
                           d_desc, d_tile_map);
    else if (U == MV_U_HUGE)
        hipLaunchKernelGGL(k_q8_matvec_multi<MV_U_HUGE>, dim3((unsigned)n_tiles), dim3(MV_THREADS), 0, s, W, X, Y,
                           d_desc, d_tile_map);
    else
        hipLaunchKernelGGL(k_q8_matvec_multi<MV_U_WIDE>, dim3((unsigned)n_tiles), dim3(MV_THREADS), 0, s, W, X, Y,
                           d_desc, d_tile_map);
    BMK_LAUNCH_CHECK();
    return 0;
}

extern "C" int mv_launch_multi(const unsigned char* W, const float* X, float* Y, const MvDesc* d_desc,
                               const unsigned int* d_tile_map, int n_tiles, hipStream_t s) {
    return launch_multi<QF_Q8>(W, X, Y, d_desc, d_tile_map, n_tiles, s);
}

/* matmul_forward_q8_vec_multi: every Q8 matvec of one decode token (or any
 * set of independent y = W x problems) in one launch.
 * buffers {0 params int {nprob, n_tiles} (by value),
 *          1 plan: MvDesc[nprob] then uint32 tile_map[n_tiles] (read on the
 *            host to validate, and by the kernel from device memory),
 *          2 weight arena (Q8 blocks), 3 activation arena f32, 4 output arena f32}.
 * Every descriptor and tile-map entry is checked against the arena sizes
 * before anything is launched. */
extern "C" int bm_q8_bmv_tiles(int OC, int C);

template <int QF>
static int launch_matvec_multi(const bmk_launch_t* a) {
    const int BYTES = QFmt<QF>::BYTES;
    BMK_NEED_BYTES(a, 0, 8, "params");
    const int nprob = bmk_pi(a, 0, 0), n_tiles = bmk_pi(a, 0, 1);
    /* optional third parameter: rows per problem (BT >= 2: the batched kernel, plan from bm_q8_bmv_plan) */
    const int BT = a->bytes[0] >= 12 ? bmk_pi(a, 0, 2) : 1;
    BMK_REQUIRE(nprob >= 0 && n_tiles >= 0, "q8 matvec multi: bad counts nprob=%d n_tiles=%d", nprob, n_tiles);
    BMK_REQUIRE(BT >= 1 && BT <= DEC_MAX_B, "q8 matvec multi: BT=%d outside [1, %d]", BT, DEC_MAX_B);
    if (nprob == 0 || n_tiles == 0) return 0;
    const size_t desc_bytes = (size_t)nprob * sizeof(MvDesc);
    BMK_NEED_BYTES(a, 1, desc_bytes + (size_t)n_tiles * 4, "plan");
    BMK_REQUIRE(((uintptr_t)a->dev[1] & 7) == 0 && ((uintptr_t)a->val[1] & 7) == 0, "q8 matvec multi: plan offset must be 8-byte aligned");
    BMK_REQUIRE(((uintptr_t)a->dev[2] & 3) == 0 && ((uintptr_t)a->dev[3] & 3) == 0 && ((uintptr_t)a->dev[4] & 3) == 0,
                "q8 matvec multi: misaligned arena offset");
    const MvDesc* desc = (const MvDesc*)a->val[1];
    const unsigned int* tmap = (const unsigned int*)((const char*)a->val[1] + desc_bytes);
    /* rows in flight per lane, as bm_q8_mv_plan chose them: MV_U_HUGE when the
     * problems take at least MV_HUGE_MIN_TILES workgroups at MV_U_WIDE */
    int U = QF == QF_Q4 ? MV_U_Q4 : MV_U_WIDE;
    if (QF == QF_Q8 && BT == 1) {
        long wide = 0;
        for (int i = 0; i < nprob; i++) {
            BMK_REQUIRE(desc[i].OC > 0 && desc[i].C > 0 && desc[i].C % 32 == 0,
                        "q8 matvec multi: problem %d bad shape OC=%d C=%d", i, desc[i].OC, desc[i].C);
            wide += mv_tiles_for(desc[i].OC, desc[i].C, MV_U_WIDE);
        }
        if (wide >= MV_HUGE_MIN_TILES) U = MV_U_HUGE;
    }
    long next_tile = 0;
    for (int i = 0; i < nprob; i++) {
        const MvDesc& d = desc[i];
        BMK_REQUIRE(d.OC > 0 && d.C > 0 && d.C % 32 == 0, "q8 matvec multi: problem %d bad shape OC=%d C=%d", i, d.OC, d.C);
        const int want = BT > 1 ? bm_q8_bmv_tiles(d.OC, d.C) : mv_tiles_for(d.OC, d.C, U);
        BMK_REQUIRE(d.tiles == want && d.tile0 == next_tile, "q8 matvec multi: problem %d tiles %d@%d, expected %d@%ld",
                    i, d.tiles, d.tile0, want, next_tile);
        BMK_REQUIRE((d.w_off & 3) == 0, "q8 matvec multi: problem %d weight offset not 4-byte aligned", i);
        /* the batched kernel loads activations 16 bytes at a time */
        BMK_REQUIRE(BT == 1 || (d.x_off & 3) == 0, "q8 matvec multi: problem %d activation offset not 16-byte aligned", i);
        BMK_REQUIRE(d.w_off + (unsigned long long)d.OC * (d.C / 32) * BYTES <= a->bytes[2] &&
                    d.x_off + (unsigned long long)BT * d.C <= a->bytes[3] / 4 &&
                    d.y_off + (unsigned long long)BT * d.OC <= a->bytes[4] / 4,
                    "q8 matvec multi: problem %d lies outside its arenas", i);
        next_tile += d.tiles;
    }
    BMK_REQUIRE(next_tile == n_tiles, "q8 matvec multi: tiles sum to %ld, n_tiles=%d", next_tile, n_tiles);
    for (int i = 0; i < nprob; i++)
        for (int t = desc[i].tile0; t < desc[i].tile0 + desc[i].tiles; t++)
            BMK_REQUIRE(tmap[t] == (unsigned)i, "q8 matvec multi: tile_map[%d]=%u, expected %d", t, tmap[t], i);
    if (BT > 1) {
        BMK_REQUIRE(((uintptr_t)a->dev[3] & 15) == 0, "q8 matvec multi: activation arena not 16-byte aligned");
        BMK_REQUIRE(launch_bmv_multi(QF, (const unsigned char*)a->dev[2], (const float*)a->dev[3], (float*)a->dev[4],
                                     (const MvDesc*)a->dev[1], (const unsigned int*)((const char*)a->dev[1] + desc_bytes),
                                     n_tiles, BT, a->stream) == 0,
                    "q8 matvec multi: batched launch failed (BT=%d)", BT);
        return 0;
    }
    return launch_multi<QF>((const unsigned char*)a->dev[2], (const float*)a->dev[3], (float*)a->dev[4],
                            (const MvDesc*)a->dev[1], (const unsigned int*)((const char*)a->dev[1] + desc_bytes),
                            n_tiles, a->stream, U);
}

extern "C" int bmk_launch_q8_matvec_multi(const bmk_launch_t* a) { return launch_matvec_multi<QF_Q8>(a); }
extern "C" int bmk_launch_q4_matvec_multi(const bmk_launch_t* a) { return launch_matvec_multi<QF_Q4>(a); }

extern "C" int dec_launch_mv(const DecMv* a, hipStream_t s);

/* matmul_forward_q8_vec / matmul_forward_q8 with BT below the GEMM cut-over:
 * buffers {inp f32 [BT][C], weight q8 [OC][C/32], bias f32 [OC], out f32 [BT][OC],
 * params int {BT, C, OC, has_bias}}.  The Metal grid (OC*128 or OC rounded to
 * 32, BT) is not needed: the launch shape follows from the parameters. */
template <int QF>
static int launch_matvec(const bmk_launch_t* a) {
    const int BYTES = QFmt<QF>::BYTES;
    BMK_NEED_BYTES(a, 4, 16, "params");
    const int BT = bmk_pi(a, 4, 0), C = bmk_pi(a, 4, 1), OC = bmk_pi(a, 4, 2), has_bias = bmk_pi(a, 4, 3);
    BMK_REQUIRE(BT >= 0 && OC >= 0 && C > 0 && C % 32 == 0, "q%d matvec: bad shape BT=%d C=%d OC=%d",
                QF == QF_Q4 ? 4 : 8, BT, C, OC);
    if (BT == 0 || OC == 0) return 0;
    BMK_NEED_BYTES(a, 0, (size_t)BT * C * 4, "inp");
    BMK_NEED_BYTES(a, 1, (size_t)OC * (C / 32) * BYTES, "weight");
    if (has_bias) BMK_NEED_BYTES(a, 2, (size_t)OC * 4, "bias");
    BMK_NEED_BYTES(a, 3, (size_t)BT * OC * 4, "out");
    BMK_REQUIRE(((uintptr_t)a->dev[0] & 3) == 0 && ((uintptr_t)a->dev[1] & 3) == 0 && ((uintptr_t)a->dev[3] & 3) == 0,
                "q8 matvec: misaligned buffer offset");
    if (BT >= 2 && BT <= DEC_MAX_B && !has_bias && ((uintptr_t)a->dev[0] & 15) == 0) {
        /* several rows: the batched fp32-MFMA matvec (decode.hip) reads each
         * weight once for all rows */
        DecMv m;
        memset(&m, 0, sizeof m);
        m.x = (const float*)a->dev[0];
        m.C = C;
        m.B = BT;
        m.ldx = C;
        m.nmat = 1;
        m.qf = QF;
        m.w[0] = (const unsigned char*)a->dev[1];
        m.y[0] = (float*)a->dev[3];
        m.OC[0] = OC;
        BMK_REQUIRE(dec_launch_mv(&m, a->stream) == 0, "q8 matvec: batched launch failed (BT=%d C=%d OC=%d)", BT, C, OC);
        return 0;
    }
    for (int bt = 0; bt < BT; bt += MV_MAX_PROBS) {
        MvGroup g;
        g.nprob = BT - bt < MV_MAX_PROBS ? BT - bt : MV_MAX_PROBS;
        for (int i = 0; i < g.nprob; i++) {
            MvProb& p = g.p[i];
            p.w = (const unsigned char*)a->dev[1];
            p.x = (const float*)a->dev[0] + (size_t)(bt + i) * C;
            p.y = (float*)a->dev[3] + (size_t)(bt + i) * OC;
            p.bias = has_bias ? (const float*)a->dev[2] : nullptr;
            p.OC = OC;
            p.nb = C / 32;
            p.tiles = 0;
        }
        if (launch_group<QF>(&g, a->stream) != 0) return -1;
    }
    return 0;
}

extern "C" int bmk_launch_q8_matvec(const bmk_launch_t* a) { return launch_matvec<QF_Q8>(a); }

/* matmul_forward_q4_vec4 / matmul_forward_q4_vec / matmul_forward_q4
 * (reference forward.metal:654-858, routing scheduler.c:755-764): the same
 * buffers over Q4_0 weights [OC][C/32] of 20-byte blocks, routed as the Q8
 * ones: one row to the matvec, 2 <= BT < 16 to the batched fp32-MFMA
 * matvec, BT >= 16 without bias to the bf16-MFMA GEMM (q8_gemm.hip). */
#include "q8_gemm.h"
#define GEMM_MIN_BT 16
extern "C" int bmk_launch_q4_matvec(const bmk_launch_t* a) {
    BMK_NEED_BYTES(a, 4, 16, "params");
    const int BT = bmk_pi(a, 4, 0), C = bmk_pi(a, 4, 1), OC = bmk_pi(a, 4, 2), has_bias = bmk_pi(a, 4, 3);
    if (BT < GEMM_MIN_BT || has_bias) return launch_matvec<QF_Q4>(a);
    BMK_REQUIRE(OC >= 0 && C > 0 && C % 32 == 0, "q4 matmul: bad shape BT=%d C=%d OC=%d", BT, C, OC);
    if (OC == 0) return 0;
    BMK_NEED_BYTES(a, 0, (size_t)BT * C * 4, "inp");
    BMK_NEED_BYTES(a, 1, (size_t)OC * (C / 32) * 20, "weight");
    BMK_NEED_BYTES(a, 3, (size_t)BT * OC * 4, "out");
    BMK_REQUIRE(((uintptr_t)a->dev[0] & 3) == 0 && ((uintptr_t)a->dev[1] & 3) == 0 && ((uintptr_t)a->dev[3] & 3) == 0,
                "q4 matmul: misaligned buffer offset");
    GmGroup g;
    g.nprob = 1;
    g.p[0].A = (const float*)a->dev[0];
    g.p[0].W = (const unsigned char*)a->dev[1];
    g.p[0].C = (float*)a->dev[3];
    g.p[0].M = BT;
    g.p[0].N = OC;
    g.p[0].K = C;
    g.p[0].lda = C;
    g.p[0].ldc = OC;
    g.p[0].tiles = 0;
    return gm_launch_group_qf(&g, 1, a->stream);
}

/* matmul_forward_q8 (reference forward.metal:625-649): BT rows of activations.
 * BT below GEMM_MIN_BT stays on fp32 (the batched fp32-MFMA matvec for
 * 2 <= BT, the matvec for one row); larger BT goes to the bf16-MFMA GEMM
 * (q8_gemm.hip). */
extern "C" int bmk_launch_q8_matmul(const bmk_launch_t* a) {
    BMK_NEED_BYTES(a, 4, 16, "params");
    const int BT = bmk_pi(a, 4, 0), C = bmk_pi(a, 4, 1), OC = bmk_pi(a, 4, 2), has_bias = bmk_pi(a, 4, 3);
    if (BT < GEMM_MIN_BT || has_bias) return bmk_launch_q8_matvec(a);
    BMK_REQUIRE(OC >= 0 && C > 0 && C % 32 == 0, "q8 matmul: bad shape BT=%d C=%d OC=%d", BT, C, OC);
    if (OC == 0) return 0;
    BMK_NEED_BYTES(a, 0, (size_t)BT * C * 4, "inp");
    BMK_NEED_BYTES(a, 1, (size_t)OC * (C / 32) * 36, "weight");
    BMK_NEED_BYTES(a, 3, (size_t)BT * OC * 4, "out");
    BMK_REQUIRE(((uintptr_t)a->dev[0] & 3) == 0 && ((uintptr_t)a->dev[1] & 3) == 0 && ((uintptr_t)a->dev[3] & 3) == 0,
                "q8 matmul: misaligned buffer offset");
    GmGroup g;
    g.nprob = 1;
    g.p[0].A = (const float*)a->dev[0];
    g.p[0].W = (const unsigned char*)a->dev[1];
    g.p[0].C = (float*)a->dev[3];
    g.p[0].M = BT;
    g.p[0].N = OC;
    g.p[0].K = C;
    g.p[0].lda = C;
    g.p[0].ldc = OC;
    g.p[0].tiles = 0;
    return gm_launch_group(&g, a->stream);
}
