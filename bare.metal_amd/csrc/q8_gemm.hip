/* SPDX-License-Identifier: MPL-2.0
 *
 * q8_gemm.hip — prefill Q8_0 GEMM on gfx950 bf16 MFMA.
 *
 *   C[m][n] = sum_k bf16(A[m][k]) * bf16(q[n][k] * scale[n][k/32])   (fp32 accumulate)
 *
 * This replaces the reference's BT > 1 path, matmul_forward_q8
 * (src/kernels/forward.metal:625-649), which computes the same sum in fp32
 * with one thread per output and no data reuse.  Operand rounding: A is cast
 * fp32 -> bf16 round-to-nearest-even, as bm_f32_to_bf16 does for finite
 * values (reference include/baremetal/types.h:22-29); each weight is
 * dequantised in fp32 (q * scale) and rounded the same way.  gfx950's
 * v_cvt_pk_bf16_f32 performs both roundings, two values per instruction.
 *
 * Tiling: a 256-lane workgroup (4 waves as 2x2) computes a 128x128 tile of
 * C; each wave owns 64x64 = 4x4 tiles of v_mfma_f32_16x16x32_bf16.  The K
 * loop steps 64 (two Q8 blocks).  LDS holds two buffers of the bf16 A slab
 * (128x64) and the dequantised weight slab (128x64), rows padded to 72
 * elements.  The global loads of step s+2 are issued before the 32 MFMAs
 * of step s, and step s+1 is converted into the other LDS buffer after
 * them: two steps of MFMA work cover each load's latency, with one
 * barrier per step.
 * Launches: up to GM_MAX_PROBS problems by value (matmul_forward_q8), or any
 * number of problems described by a device table (matmul_forward_q8_multi).
 */
#include "bmk.h"
#include "q8_gemm.h"

#include <stdlib.h>

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int BM = GM_BM, BN = GM_BN, NTH = 256;
constexpr int GEMM_BK = 64;        /* K step of the launched kernels (see gemm_tile) */
constexpr bool TWO_STAGE = false;  /* prefetch depth of the launched kernels (see gemm_tile) */
constexpr int GEMM_BK_BF16 = 64;   /* K step of the bf16-activation kernel */
constexpr bool TWO_STAGE_BF16 = true;
constexpr bool DEEP_W_BF16 = false;  /* bf16 kernel: W four steps ahead, A two */

/* LDS of one tile: 2 buffers x (A slab + W slab), rows of BK + 8 bf16 */
template <int BK>
constexpr int gemm_lds_elems() { return 4 * BM * (BK + 8); }

/* fp32 pair -> packed bf16 pair, round to nearest even (v_cvt_pk_bf16_f32) */
__device__ __forceinline__ unsigned int pk_bf16(float lo, float hi) {
    const f32x2 v = {lo, hi};
    const bf16x2 r = __builtin_convertvector(v, bf16x2);
    unsigned int u;
    __builtin_memcpy(&u, &r, 4);
    return u;
}

__device__ __forceinline__ float sbyte(unsigned int w, int k) { return (float)(signed char)((w >> (8 * k)) & 0xffu); }

/* One K step of one loader thread (BK = 64: two Q8 blocks, BK = 32: one).
 * A (fp32): rows t/(BK/4) + (1024/BK)*p (p < BK/8), columns 4*(t % (BK/4))
 * .. +4; A (bf16): rows t/(BK/8) + (2048/BK)*p (p < BK/16), columns
 * 8*(t % (BK/8)) .. +8.  Either way the lanes of a row read it
 * contiguously and a wave instruction covers whole rows.  W: row t/2;
 * BK = 64: Q8 block 2*step + t%2 (36 bytes), BK = 32: half t%2 of the
 * step's block (scale + 16 bytes). */
template <int BK, bool ABF16>
struct Stage {
    float4 a[ABF16 ? 1 : BK / 8];
    uint4 ab[ABF16 ? BK / 16 : 1];
    float s;
    uint4 q[BK / 32];
};

__device__ __forceinline__ uint4 dq8(const uint4& q, int half, float s) {
    const unsigned int w0 = half ? q.z : q.x, w1 = half ? q.w : q.y;
    uint4 r;
    r.x = pk_bf16(sbyte(w0, 0) * s, sbyte(w0, 1) * s);
    r.y = pk_bf16(sbyte(w0, 2) * s, sbyte(w0, 3) * s);
    r.z = pk_bf16(sbyte(w1, 0) * s, sbyte(w1, 1) * s);
    r.w = pk_bf16(sbyte(w1, 2) * s, sbyte(w1, 3) * s);
    return r;
}

/* One 128x128 tile of C.  lds: 2 buffers x (A slab + W slab).
 * DEPTH2 = false: per K step s, issue the global loads of step s+1, run the
 * MFMAs of step s from LDS, convert step s+1 into the other buffer,
 * barrier.  DEPTH2 = true: two register stages; the loads of step s+2 are
 * issued before the MFMAs of step s. */
template <int BK, bool DEPTH2, bool ABF16, bool DEEPW = false>
__device__ __forceinline__ void gemm_tile(const void* __restrict__ Av, const unsigned char* __restrict__ W,
                                          float* __restrict__ Cm, int M, int N, int K, int lda, int ldc, int tm,
                                          int tn, unsigned short* lds) {
    constexpr int LDK = BK + 8;
    constexpr int SLAB = BM * LDK;
    constexpr int CPR = ABF16 ? BK / 8 : BK / 4; /* 16-byte chunks of an A row */
    constexpr int RPP = NTH / CPR;               /* A rows per loader pass */
    constexpr int NPASS = BM / RPP;              /* BK/16 (bf16) or BK/8 (fp32) */
    constexpr int EPC = ABF16 ? 8 : 4;           /* A elements per chunk */
    const int t = threadIdx.x;
    const int wave = t >> 6, lane = t & 63;
    const int wm = (wave >> 1) * 64, wn = (wave & 1) * 64;
    const int m0 = tm * BM, n0 = tn * BN;
    const int nb = K / 32;
    const int nsteps = (K + BK - 1) / BK;
    const int lr = t >> 1, lh = t & 1;           /* W loader: row, half */
    const int ar = t / CPR, ac = t % CPR;        /* A loader: first row, float4 column */
    /* Rows past M (or N) only feed C entries that are never stored, so the
     * loaders clamp them to the last row instead of branching; only a K
     * block past the end (odd block count with BK = 64) must contribute
     * zero, which the selects below provide.  Offsets are 32-bit from
     * workgroup-uniform bases (the launchers check that they fit). */
    const float* Af = (const float*)Av + (ABF16 ? 0 : (size_t)m0 * lda);
    const unsigned short* Ah = (const unsigned short*)Av + (ABF16 ? (size_t)m0 * lda : 0);
    const unsigned char* Wb = W + (size_t)n0 * nb * 36;
    unsigned int aoff[NPASS];
#pragma unroll
    for (int p = 0; p < NPASS; p++) aoff[p] = (unsigned)min(ar + RPP * p, M - 1 - m0) * (unsigned)lda + (unsigned)(EPC * ac);
    const unsigned int woff = (unsigned)min(lr, N - 1 - n0) * (unsigned)(nb * 36);

    /* split loaders for the deep-W pipeline: A stages and W stages rotate separately */
    auto load_a = [&](int step, Stage<BK, ABF16>& st) {
        const bool ka = (BK * step + EPC * ac) / 32 < nb;
        const unsigned int col = ka ? (unsigned)(step * BK) : 0u;
#pragma unroll
        for (int p = 0; p < NPASS; p++) {
            if (ABF16) {
                uint4 v;
                __builtin_memcpy(&v, __builtin_assume_aligned(Ah + aoff[p] + col, 4), 16);
                st.ab[p] = ka ? v : make_uint4(0, 0, 0, 0);
            } else {
                float4 v;
                __builtin_memcpy(&v, __builtin_assume_aligned(Af + aoff[p] + col, 4), 16);
                st.a[p] = ka ? v : make_float4(0.f, 0.f, 0.f, 0.f);
            }
        }
    };
    auto load_w = [&](int step, Stage<BK, ABF16>& st) {
        const int kb = BK == 64 ? 2 * step + lh : step;
        const bool kw = kb < nb;
        const unsigned char* blk = Wb + woff + (unsigned)(kw ? kb : 0) * 36u;
        float sc;
        __builtin_memcpy(&sc, __builtin_assume_aligned(blk, 4), 4);
        if (BK == 64) {
            __builtin_memcpy(&st.q[0], __builtin_assume_aligned(blk + 4, 4), 16);
            __builtin_memcpy(&st.q[BK / 32 - 1], __builtin_assume_aligned(blk + 20, 4), 16);
        } else {
            __builtin_memcpy(&st.q[0], __builtin_assume_aligned(blk + 4 + 16 * lh, 4), 16);
        }
        st.s = kw ? sc : 0.0f;
    };
    auto load = [&](int step, Stage<BK, ABF16>& st) {
        /* column BK*step + EPC*ac lies in Q8 block (BK*step + EPC*ac) / 32 */
        const bool ka = (BK * step + EPC * ac) / 32 < nb;
        const unsigned int col = ka ? (unsigned)(step * BK) : 0u;
#pragma unroll
        for (int p = 0; p < NPASS; p++) {
            if (ABF16) {
                uint4 v;
                __builtin_memcpy(&v, __builtin_assume_aligned(Ah + aoff[p] + col, 4), 16);
                st.ab[p] = ka ? v : make_uint4(0, 0, 0, 0);
            } else {
                float4 v;
                __builtin_memcpy(&v, __builtin_assume_aligned(Af + aoff[p] + col, 4), 16);
                st.a[p] = ka ? v : make_float4(0.f, 0.f, 0.f, 0.f);
            }
        }
        const int kb = BK == 64 ? 2 * step + lh : step; /* this thread's Q8 block */
        const bool kw = kb < nb;
        const unsigned char* blk = Wb + woff + (unsigned)(kw ? kb : 0) * 36u;
        float sc;
        __builtin_memcpy(&sc, __builtin_assume_aligned(blk, 4), 4);
        if (BK == 64) {
            __builtin_memcpy(&st.q[0], __builtin_assume_aligned(blk + 4, 4), 16);
            __builtin_memcpy(&st.q[BK / 32 - 1], __builtin_assume_aligned(blk + 20, 4), 16);
        } else {
            __builtin_memcpy(&st.q[0], __builtin_assume_aligned(blk + 4 + 16 * lh, 4), 16);
        }
        st.s = kw ? sc : 0.0f; /* a zero scale turns the (finite) q into zeros */
    };
    auto store_aw = [&](int buf, const Stage<BK, ABF16>& sa, const Stage<BK, ABF16>& sw) {
        unsigned short* As = lds + buf * 2 * SLAB;
        unsigned short* Bs = As + SLAB;
#pragma unroll
        for (int p = 0; p < NPASS; p++) {
            if (ABF16) {
                *(uint4*)&As[(ar + RPP * p) * LDK + 8 * ac] = sa.ab[p];
            } else {
                uint2 v;
                v.x = pk_bf16(sa.a[p].x, sa.a[p].y);
                v.y = pk_bf16(sa.a[p].z, sa.a[p].w);
                *(uint2*)&As[(ar + RPP * p) * LDK + 4 * ac] = v;
            }
        }
        uint4* bp = (uint4*)&Bs[lr * LDK + (BK / 2) * lh];
#pragma unroll
        for (int i = 0; i < BK / 32; i++) {
            bp[2 * i] = dq8(sw.q[i], 0, sw.s);
            bp[2 * i + 1] = dq8(sw.q[i], 1, sw.s);
        }
    };
    auto store = [&](int buf, const Stage<BK, ABF16>& st) {
        unsigned short* As = lds + buf * 2 * SLAB;
        unsigned short* Bs = As + SLAB;
#pragma unroll
        for (int p = 0; p < NPASS; p++) {
            if (ABF16) {
                *(uint4*)&As[(ar + RPP * p) * LDK + 8 * ac] = st.ab[p];
            } else {
                uint2 v;
                v.x = pk_bf16(st.a[p].x, st.a[p].y);
                v.y = pk_bf16(st.a[p].z, st.a[p].w);
                *(uint2*)&As[(ar + RPP * p) * LDK + 4 * ac] = v;
            }
        }
        uint4* bp = (uint4*)&Bs[lr * LDK + (BK / 2) * lh];
#pragma unroll
        for (int i = 0; i < BK / 32; i++) {
            bp[2 * i] = dq8(st.q[i], 0, st.s);
            bp[2 * i + 1] = dq8(st.q[i], 1, st.s);
        }
    };

    f32x4 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    const int kq = (lane >> 4) * 8;
    auto mfma_step = [&](int buf) {
        const unsigned short* As = lds + buf * 2 * SLAB;
        const unsigned short* Bs = As + SLAB;
#pragma unroll
        for (int ks = 0; ks < BK; ks += 32) {
            bf16x8 fa[4], fb[4];
#pragma unroll
            for (int i = 0; i < 4; i++) fa[i] = *(const bf16x8*)&As[(wm + 16 * i + (lane & 15)) * LDK + ks + kq];
#pragma unroll
            for (int j = 0; j < 4; j++) fb[j] = *(const bf16x8*)&Bs[(wn + 16 * j + (lane & 15)) * LDK + ks + kq];
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int j = 0; j < 4; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fa[i], fb[j], acc[i][j], 0, 0, 0);
        }
    };

    if (!DEPTH2 && !DEEPW) {
        Stage<BK, ABF16> s0;
        load(0, s0);
        store(0, s0);
        __syncthreads();
        for (int step = 0; step < nsteps; step++) {
            const int cur = step & 1;
            if (step + 1 < nsteps) load(step + 1, s0);
            mfma_step(cur);
            if (step + 1 < nsteps) store(cur ^ 1, s0);
            __syncthreads();
        }
    } else if (DEEPW) {
        /* A two steps ahead (stages a0, a1), W four steps ahead (w0..w3).
         * Step s: issue A(s+2) into a[s%2] and W(s+4) into w[s%4], run the
         * MFMAs of step s, store A(s+1), W(s+1) into the other LDS buffer.
         * Unrolled by four so that every stage is named statically. */
        Stage<BK, ABF16> a0, a1, w0, w1, w2, w3;
        load_a(0, a0);
        load_w(0, w0);
        if (nsteps > 1) { load_a(1, a1); load_w(1, w1); }
        if (nsteps > 2) load_w(2, w2);
        if (nsteps > 3) load_w(3, w3);
        store_aw(0, a0, w0);
        __syncthreads();
#define GM_STEP(S, AC, AN, WC, WN)                                  \
        if ((S) < nsteps) {                                         \
            if ((S) + 2 < nsteps) load_a((S) + 2, AC);              \
            if ((S) + 4 < nsteps) load_w((S) + 4, WC);              \
            mfma_step((S) & 1);                                     \
            if ((S) + 1 < nsteps) store_aw(((S) + 1) & 1, AN, WN);  \
            __syncthreads();                                        \
        }
        for (int st4 = 0; st4 < nsteps; st4 += 4) {
            GM_STEP(st4 + 0, a0, a1, w0, w1)
            GM_STEP(st4 + 1, a1, a0, w1, w2)
            GM_STEP(st4 + 2, a0, a1, w2, w3)
            GM_STEP(st4 + 3, a1, a0, w3, w0)
        }
#undef GM_STEP
    } else {
        Stage<BK, ABF16> s0, s1;
        load(0, s0);
        if (nsteps > 1) load(1, s1);
        store(0, s0);
        __syncthreads();
        int step = 0;
        /* steps two at a time so that the register stages are named statically */
        for (; step + 2 <= nsteps; step += 2) {
            if (step + 2 < nsteps) load(step + 2, s0); /* s0 is free: step's data is in LDS buffer 0 */
            mfma_step(0);
            store(1, s1);
            __syncthreads();
            if (step + 3 < nsteps) load(step + 3, s1);
            mfma_step(1);
            if (step + 2 < nsteps) store(0, s0);
            __syncthreads();
        }
        if (step < nsteps) mfma_step(0); /* odd step count: the last step sits in buffer 0 */
    }

    /* D layout of a 16x16 MFMA tile: lane holds rows 4*(lane/16)+v, column lane%16 */
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int col = n0 + wn + 16 * j + (lane & 15);
            if (col >= N) continue;
#pragma unroll
            for (int v = 0; v < 4; v++) {
                const int row = m0 + wm + 16 * i + (lane >> 4) * 4 + v;
                if (row < M) Cm[(size_t)row * ldc + col] = acc[i][j][v];
            }
        }
}

__global__ __launch_bounds__(NTH) void k_q8_gemm(GmGroup g) {
    __shared__ __attribute__((aligned(16))) unsigned short lds[gemm_lds_elems<GEMM_BK>()];
    int tile = blockIdx.x;
    int pi = 0;
    while (pi + 1 < g.nprob && tile >= g.p[pi].tiles) {
        tile -= g.p[pi].tiles;
        pi++;
    }
    const GmProb& p = g.p[pi];
    const int tiles_n = (p.N + BN - 1) / BN;
    gemm_tile<GEMM_BK, TWO_STAGE, false>(p.A, p.W, p.C, p.M, p.N, p.K, p.lda, p.ldc, tile / tiles_n, tile % tiles_n,
                                         lds);
}

/* Activations in fp32 (cast to bf16 while staging) or already in bf16. */
template <bool ABF16>
__global__ __launch_bounds__(NTH) void k_q8_gemm_multi(const void* __restrict__ A, const unsigned char* __restrict__ W,
                                                       float* __restrict__ C, const GmDesc* __restrict__ desc,
                                                       const unsigned int* __restrict__ tile_map) {
    constexpr int BKM = ABF16 ? GEMM_BK_BF16 : GEMM_BK;
    __shared__ __attribute__((aligned(16))) unsigned short lds[gemm_lds_elems<BKM>()];
    const unsigned int tm_ = tile_map[blockIdx.x];
    if (tm_ == GM_IDLE_TILE) return;
    const GmDesc d = desc[tm_ >> 16];
    const int tile = (int)(tm_ & 0xffffu);
    const int tiles_n = (d.N + BN - 1) / BN;
    const void* Ad = ABF16 ? (const void*)((const unsigned short*)A + d.a_off) : (const void*)((const float*)A + d.a_off);
    gemm_tile<BKM, ABF16 ? TWO_STAGE_BF16 : TWO_STAGE, ABF16, ABF16 && DEEP_W_BF16>(
        Ad, W + d.w_off, C + d.c_off, d.M, d.N, d.K, d.lda, d.ldc, tile / tiles_n, tile % tiles_n, lds);
}

/* fp32 -> bf16 (round to nearest even), 8 elements per lane */
__global__ __launch_bounds__(NTH) void k_cast_bf16(const float* __restrict__ src, unsigned short* __restrict__ dst,
                                                   long n8, long n) {
    const long i = (long)blockIdx.x * NTH + threadIdx.x;
    if (i < n8) {
        float4 a, b;
        __builtin_memcpy(&a, src + 8 * i, 16);
        __builtin_memcpy(&b, src + 8 * i + 4, 16);
        uint4 v;
        v.x = pk_bf16(a.x, a.y);
        v.y = pk_bf16(a.z, a.w);
        v.z = pk_bf16(b.x, b.y);
        v.w = pk_bf16(b.z, b.w);
        __builtin_memcpy(dst + 8 * i, &v, 16);
    } else if (i == n8) {
        for (long j = 8 * n8; j < n; j++) dst[j] = (unsigned short)(pk_bf16(src[j], 0.0f) & 0xffffu);
    }
}

} // namespace

extern "C" int gm_tiles_for(int M, int N) { return ((M + BM - 1) / BM) * ((N + BN - 1) / BN); }

/* The tile loaders address a problem with 32-bit offsets. */
static bool gm_offsets_fit(int M, int N, int K, int lda) {
    return (unsigned long long)M * (unsigned long long)lda < 0x80000000ull &&
           (unsigned long long)N * (unsigned long long)(K / 32) * 36ull < 0x80000000ull;
}

extern "C" int gm_launch_group(GmGroup* g, hipStream_t s) {
    long total = 0;
    for (int i = 0; i < g->nprob; i++)
        BMK_REQUIRE(gm_offsets_fit(g->p[i].M, g->p[i].N, g->p[i].K, g->p[i].lda),
                    "q8 gemm: problem %d too large for 32-bit tile offsets", i);
    for (int i = 0; i < g->nprob; i++) {
        g->p[i].tiles = gm_tiles_for(g->p[i].M, g->p[i].N);
        total += g->p[i].tiles;
    }
    if (total <= 0) return 0;
    hipLaunchKernelGGL(k_q8_gemm, dim3((unsigned)total), dim3(NTH), 0, s, *g);
    BMK_LAUNCH_CHECK();
    return 0;
}

/* matmul_forward_q8_multi: many independent prefill GEMMs in one launch.
 * buffers {0 params int {nprob, n_tiles[, a_bf16]} (by value; a_bf16 = 1: the
 *            activation arena holds bf16, offsets and strides in elements),
 *          1 plan: GmDesc[nprob] then uint32 tile_map[n_tiles] = (problem << 16) | tile
 *            (host-validated: a permutation of all tiles; read by the kernel),
 *          2 activation arena f32, 3 weight arena (Q8 blocks), 4 output arena f32}. */
extern "C" int bmk_launch_q8_gemm_multi(const bmk_launch_t* a) {
    BMK_NEED_BYTES(a, 0, 8, "params");
    const int nprob = bmk_pi(a, 0, 0), n_tiles = bmk_pi(a, 0, 1);
    const int a_bf16 = a->bytes[0] >= 12 ? bmk_pi(a, 0, 2) : 0;
    const unsigned long long esz = a_bf16 ? 2 : 4; /* bytes per activation element */
    BMK_REQUIRE(nprob >= 0 && n_tiles >= 0 && (a_bf16 == 0 || a_bf16 == 1),
                "q8 gemm multi: bad params nprob=%d n_tiles=%d a_bf16=%d", nprob, n_tiles, a_bf16);
    if (nprob == 0 || n_tiles == 0) return 0;
    const size_t desc_bytes = (size_t)nprob * sizeof(GmDesc);
    BMK_NEED_BYTES(a, 1, desc_bytes + (size_t)n_tiles * 4, "plan");
    BMK_REQUIRE(((uintptr_t)a->dev[1] & 7) == 0 && ((uintptr_t)a->val[1] & 7) == 0,
                "q8 gemm multi: plan offset must be 8-byte aligned");
    BMK_REQUIRE(((uintptr_t)a->dev[2] & 3) == 0 && ((uintptr_t)a->dev[3] & 3) == 0 && ((uintptr_t)a->dev[4] & 3) == 0,
                "q8 gemm multi: misaligned arena offset");
    const GmDesc* desc = (const GmDesc*)a->val[1];
    const unsigned int* tmap = (const unsigned int*)((const char*)a->val[1] + desc_bytes);
    long next_tile = 0;
    for (int i = 0; i < nprob; i++) {
        const GmDesc& d = desc[i];
        BMK_REQUIRE(d.M > 0 && d.N > 0 && d.K > 0 && d.K % 32 == 0 && d.lda >= d.K && d.ldc >= d.N,
                    "q8 gemm multi: problem %d bad shape M=%d N=%d K=%d lda=%d ldc=%d", i, d.M, d.N, d.K, d.lda, d.ldc);
        BMK_REQUIRE(d.tiles == gm_tiles_for(d.M, d.N) && d.tile0 == next_tile,
                    "q8 gemm multi: problem %d tiles %d@%d, expected %d@%ld", i, d.tiles, d.tile0,
                    gm_tiles_for(d.M, d.N), next_tile);
        BMK_REQUIRE((d.w_off & 3) == 0, "q8 gemm multi: problem %d weight offset not 4-byte aligned", i);
        BMK_REQUIRE(gm_offsets_fit(d.M, d.N, d.K, d.lda), "q8 gemm multi: problem %d too large for 32-bit tile offsets",
                    i);
        BMK_REQUIRE((!a_bf16 || (d.a_off % 8 == 0 && d.lda % 8 == 0)),
                    "q8 gemm multi: problem %d bf16 rows must start 16-byte aligned", i);
        BMK_REQUIRE(d.a_off + (unsigned long long)(d.M - 1) * d.lda + d.K <= a->bytes[2] / esz &&
                        d.w_off + (unsigned long long)d.N * (d.K / 32) * 36 <= a->bytes[3] &&
                        d.c_off + (unsigned long long)(d.M - 1) * d.ldc + d.N <= a->bytes[4] / 4,
                    "q8 gemm multi: problem %d lies outside its arenas", i);
        next_tile += d.tiles;
    }
    BMK_REQUIRE(next_tile <= n_tiles, "q8 gemm multi: %ld tiles do not fit %d workgroups", next_tile, n_tiles);
    BMK_REQUIRE(nprob <= 0xffff, "q8 gemm multi: %d problems, at most 65535", nprob);
    /* tile_map must name every (problem, tile) exactly once; the rest are idle */
    unsigned char* seen = (unsigned char*)calloc((size_t)next_tile + 1, 1);
    BMK_REQUIRE(seen != nullptr, "q8 gemm multi: out of host memory");
    long named = 0;
    for (int b = 0; b < n_tiles; b++) {
        if (tmap[b] == GM_IDLE_TILE) continue;
        named++;
        const unsigned int p = tmap[b] >> 16, tl = tmap[b] & 0xffffu;
        const bool ok = p < (unsigned)nprob && tl < (unsigned)desc[p].tiles && !seen[desc[p].tile0 + tl];
        if (!ok) {
            free(seen);
            BMK_ERR("q8 gemm multi: tile_map[%d] = problem %u tile %u is out of range or repeated", b, p, tl);
            return -1;
        }
        seen[desc[p].tile0 + tl] = 1;
    }
    free(seen);
    BMK_REQUIRE(named == next_tile, "q8 gemm multi: tile_map names %ld of %ld tiles", named, next_tile);
    const GmDesc* dd = (const GmDesc*)a->dev[1];
    const unsigned int* dt = (const unsigned int*)((const char*)a->dev[1] + desc_bytes);
    if (a_bf16) {
        BMK_REQUIRE(((uintptr_t)a->dev[2] & 15) == 0, "q8 gemm multi: bf16 activation arena must be 16-byte aligned");
        hipLaunchKernelGGL(k_q8_gemm_multi<true>, dim3((unsigned)n_tiles), dim3(NTH), 0, a->stream,
                           (const void*)a->dev[2], (const unsigned char*)a->dev[3], (float*)a->dev[4], dd, dt);
    } else {
        hipLaunchKernelGGL(k_q8_gemm_multi<false>, dim3((unsigned)n_tiles), dim3(NTH), 0, a->stream,
                           (const void*)a->dev[2], (const unsigned char*)a->dev[3], (float*)a->dev[4], dd, dt);
    }
    BMK_LAUNCH_CHECK();
    return 0;
}

/* cast_f32_bf16 {src f32 [n], dst bf16 [n], params int64{n}}: round to nearest even,
 * the activation cast of a prefill GEMM done once per matrix. */
extern "C" int bmk_launch_cast_bf16(const bmk_launch_t* a) {
    BMK_NEED_BYTES(a, 2, 8, "params");
    long long n;
    __builtin_memcpy(&n, a->val[2], 8);
    BMK_REQUIRE(n >= 0, "cast_f32_bf16: negative count");
    if (n == 0) return 0;
    BMK_NEED_BYTES(a, 0, (size_t)n * 4, "src");
    BMK_NEED_BYTES(a, 1, (size_t)n * 2, "dst");
    BMK_REQUIRE(((uintptr_t)a->dev[0] & 15) == 0 && ((uintptr_t)a->dev[1] & 15) == 0,
                "cast_f32_bf16: operands must be 16-byte aligned");
    const long n8 = (long)(n / 8);
    const long threads = n8 + 1;
    hipLaunchKernelGGL(k_cast_bf16, dim3((unsigned)((threads + NTH - 1) / NTH)), dim3(NTH), 0, a->stream,
                       (const float*)a->dev[0], (unsigned short*)a->dev[1], n8, (long)n);
    BMK_LAUNCH_CHECK();
    return 0;
}
