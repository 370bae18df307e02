/* SPDX-License-Identifier: MPL-2.0
 *
 * q8_gemm.hip — prefill Q8_0 GEMM on gfx950 bf16 MFMA.
 *
 *   C[m][n] = sum_k bf16(A[m][k]) * bf16(q[n][k] * scale[n][k/32])   (fp32 accumulate)
 *
 * This replaces the reference's BT > 1 path, matmul_forward_q8
 * (src/kernels/forward.metal:625-649), which computes the same sum in fp32
 * with one thread per output and no data reuse.  Operand rounding: A is cast
 * fp32 -> bf16 round-to-nearest-even exactly as bm_f32_to_bf16 does
 * (reference include/baremetal/types.h:22-29, bit trick, no NaN special
 * case); each weight is dequantised in fp32 (q * scale) and then rounded the
 * same way.
 *
 * Tiling: a 256-lane workgroup (4 waves as 2x2) computes a 64x64 tile of C;
 * each wave owns 32x32 = 2x2 MFMA 16x16 tiles.  The K loop steps one Q8
 * block (32) at a time: the A slab (64x32 fp32) and the 64 weight blocks are
 * loaded into registers one step ahead, converted/dequantised to bf16 and
 * written to LDS, then every wave issues 4 v_mfma_f32_16x16x32_bf16.  LDS
 * rows are padded to 40 bf16 to spread the 16-byte reads over banks.
 * Up to GM_MAX_PROBS independent GEMMs share a launch (q/k/v/o/gate/up/down
 * of a layer when their inputs are independent).
 */
#include "bmk.h"
#include "q8_gemm.h"

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int BM = 64, BN = 64, BK = 32, LDK = BK + 8;

__device__ __forceinline__ unsigned short bf16_rne_bits(float f) {
    unsigned int u = __float_as_uint(f);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (unsigned short)(u >> 16);
}

__device__ __forceinline__ unsigned int pack2(float lo, float hi) {
    return (unsigned int)bf16_rne_bits(lo) | ((unsigned int)bf16_rne_bits(hi) << 16);
}

__device__ __forceinline__ float sbyte(unsigned int w, int k) { return (float)(signed char)((w >> (8 * k)) & 0xffu); }

__global__ __launch_bounds__(256) void k_q8_gemm(GmGroup g) {
    __shared__ __attribute__((aligned(16))) unsigned short As[BM * LDK];
    __shared__ __attribute__((aligned(16))) unsigned short Bs[BN * LDK];

    int tile = blockIdx.x;
    int pi = 0;
    while (pi + 1 < g.nprob && tile >= g.p[pi].tiles) {
        tile -= g.p[pi].tiles;
        pi++;
    }
    const GmProb& p = g.p[pi];
    const int tiles_n = (p.N + BN - 1) / BN;
    const int m0 = (tile / tiles_n) * BM;
    const int n0 = (tile % tiles_n) * BN;
    const int nb = p.K / 32;

    const int t = threadIdx.x;
    const int lr = t >> 2;        /* row of the slab this lane loads (0..63) */
    const int lc = (t & 3) * 8;   /* first k of the 8 it loads */
    const int wave = t >> 6, lane = t & 63;
    const int wm = (wave >> 1) * 32, wn = (wave & 1) * 32;

    const bool a_ok = (m0 + lr) < p.M;
    const bool b_ok = (n0 + lr) < p.N;
    const float* arow = p.A + (size_t)(m0 + lr) * p.lda + lc;
    const unsigned char* brow = p.W + (size_t)(n0 + lr) * nb * 36;

    f32x4 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    float4 ra0, ra1;
    float rs;
    uint2 rq;
    auto load_step = [&](int kb) {
        if (a_ok) {
            __builtin_memcpy(&ra0, __builtin_assume_aligned(arow + kb * 32, 4), 16);
            __builtin_memcpy(&ra1, __builtin_assume_aligned(arow + kb * 32 + 4, 4), 16);
        } else {
            ra0 = make_float4(0.f, 0.f, 0.f, 0.f);
            ra1 = ra0;
        }
        if (b_ok) {
            const unsigned char* blk = brow + (size_t)kb * 36;
            __builtin_memcpy(&rs, __builtin_assume_aligned(blk, 4), 4);
            __builtin_memcpy(&rq, __builtin_assume_aligned(blk + 4 + lc, 4), 8);
        } else {
            rs = 0.f;
            rq = make_uint2(0, 0);
        }
    };

    load_step(0);
    for (int kb = 0; kb < nb; kb++) {
        /* registers -> bf16 -> LDS */
        uint4 av, bv;
        av.x = pack2(ra0.x, ra0.y); av.y = pack2(ra0.z, ra0.w);
        av.z = pack2(ra1.x, ra1.y); av.w = pack2(ra1.z, ra1.w);
        bv.x = pack2(sbyte(rq.x, 0) * rs, sbyte(rq.x, 1) * rs);
        bv.y = pack2(sbyte(rq.x, 2) * rs, sbyte(rq.x, 3) * rs);
        bv.z = pack2(sbyte(rq.y, 0) * rs, sbyte(rq.y, 1) * rs);
        bv.w = pack2(sbyte(rq.y, 2) * rs, sbyte(rq.y, 3) * rs);
        __syncthreads(); /* previous step's MFMA reads are done */
        *(uint4*)&As[lr * LDK + lc] = av;
        *(uint4*)&Bs[lr * LDK + lc] = bv;
        __syncthreads();
        if (kb + 1 < nb) load_step(kb + 1);

        const int kq = (lane >> 4) * 8;
        bf16x8 fa[2], fb[2];
#pragma unroll
        for (int i = 0; i < 2; i++) {
            const int r = wm + i * 16 + (lane & 15);
            fa[i] = *(const bf16x8*)&As[r * LDK + kq];
        }
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const int c = wn + j * 16 + (lane & 15);
            fb[j] = *(const bf16x8*)&Bs[c * LDK + kq];
        }
#pragma unroll
        for (int i = 0; i < 2; i++)
#pragma unroll
            for (int j = 0; j < 2; j++)
                acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fa[i], fb[j], acc[i][j], 0, 0, 0);
    }

    /* D layout of a 16x16 MFMA tile: lane holds rows 4*(lane/16)+v, column lane%16 */
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const int col = n0 + wn + j * 16 + (lane & 15);
            if (col >= p.N) continue;
#pragma unroll
            for (int v = 0; v < 4; v++) {
                const int row = m0 + wm + i * 16 + (lane >> 4) * 4 + v;
                if (row < p.M) p.C[(size_t)row * p.ldc + col] = acc[i][j][v];
            }
        }
}

} // namespace

extern "C" int gm_tiles_for(int M, int N) { return ((M + BM - 1) / BM) * ((N + BN - 1) / BN); }

extern "C" int gm_launch_group(GmGroup* g, hipStream_t s) {
    long total = 0;
    for (int i = 0; i < g->nprob; i++) {
        g->p[i].tiles = gm_tiles_for(g->p[i].M, g->p[i].N);
        total += g->p[i].tiles;
    }
    if (total <= 0) return 0;
    hipLaunchKernelGGL(k_q8_gemm, dim3((unsigned)total), dim3(256), 0, s, *g);
    BMK_LAUNCH_CHECK();
    return 0;
}
