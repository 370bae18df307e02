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
 * C; each wave owns 64x64 = 2x2 tiles of v_mfma_f32_32x32x16_bf16.  The K
 * loop steps 64 (two Q8 blocks).  LDS holds two buffers of the bf16 A slab
 * (128x64) and the dequantised weight slab (128x64), rows padded to 72
 * elements.  The global loads of step s+2 are issued before the 16 MFMAs
 * of step s, and step s+1 is converted into the other LDS buffer after
 * them: two steps of MFMA work cover each load's latency, with one
 * barrier per step (details at gemm_tile).
 * Launches: up to GM_MAX_PROBS problems by value (matmul_forward_q8), or any
 * number of problems described by a device table (matmul_forward_q8_multi).
 */
#include "bmk.h"
#include "q8_gemm.h"
#include "q8_common.h"

#include <stdlib.h>

namespace {

using bmk::QFmt;
using bmk::QF_Q8;
using bmk::QF_Q4;
using bmk::q4_code;

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int BM = GM_BM, BN = GM_BN, NTH = 256;
constexpr int GEMM_BK = 64;         /* K step: two Q8 blocks */
constexpr int LDK = GEMM_BK + 8;    /* LDS row in bf16 elements; the padding spreads rows over the banks */
constexpr int SLAB = BM * LDK;      /* one operand slab (BM == BN) */
constexpr int GEMM_LDS = 4 * SLAB;  /* 2 buffers x (A slab + W slab), bf16 elements */

/* fp32 pair -> packed bf16 pair, round to nearest even (v_cvt_pk_bf16_f32) */
__device__ __forceinline__ unsigned int pk_bf16(float lo, float hi) {
    const f32x2 v = {lo, hi};
    const bf16x2 r = __builtin_convertvector(v, bf16x2);
    unsigned int u;
    __builtin_memcpy(&u, &r, 4);
    return u;
}

__device__ __forceinline__ float sbyte(unsigned int w, int k) { return (float)(signed char)((w >> (8 * k)) & 0xffu); }

/* Register stage of one loader thread for one K step (two Q8 blocks).
 * A (fp32): rows t/16 + 16p (p < 8), columns 4*(t%16) .. +4; A (bf16):
 * rows t/8 + 32p (p < 4), columns 8*(t%8) .. +8.  Either way the lanes of a
 * row read it contiguously and a wave instruction covers whole rows.
 * W: row t/2, Q8 block 2*step + t%2 (36 bytes: scale, 32 int8). */
template <bool ABF16, int QF = QF_Q8>
struct Stage {
    float4 a[ABF16 ? 1 : 8];
    uint4 ab[ABF16 ? 4 : 1];
    float s;
    uint4 q[QF == QF_Q4 ? 1 : 2]; /* the block's 32 codes: int8 (Q8_0) or nibbles (Q4_0) */
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

/* 8 Q4_0 codes (dword `part` of the block's 16 code bytes), each
 * times the scale and rounded to bf16, as 8 packed bf16 */
__device__ __forceinline__ uint4 dq4(const uint4& q, int part, float s) {
    const unsigned int w = part == 0 ? q.x : part == 1 ? q.y : part == 2 ? q.z : q.w;
    uint4 r;
    r.x = pk_bf16(q4_code(w, 0) * s, q4_code(w, 1) * s);
    r.y = pk_bf16(q4_code(w, 2) * s, q4_code(w, 3) * s);
    r.z = pk_bf16(q4_code(w, 4) * s, q4_code(w, 5) * s);
    r.w = pk_bf16(q4_code(w, 6) * s, q4_code(w, 7) * s);
    return r;
}

/* One 128x128 tile of C; lds holds 2 buffers x (A slab + W slab).
 *
 * K runs in steps of 64 (two Q8 blocks).  The nb/2 full steps form a
 * two-stage pipeline: the global loads of step s+2 are issued before the
 * 16 MFMAs of step s, and step s+1 is stored into the other LDS buffer
 * after them, with one barrier per step.  The loop body has no data
 * dependent selects and issues the same loads on every path (past the
 * last step it reloads that step, an L2 hit that is never stored), so the
 * compiler's wait before a store counts only the loads that feed it; a
 * conditional load or an early consumer of a load's registers makes it
 * drain the whole queue instead.  An odd block count leaves a half step,
 * run after the loop with the out-of-range half zeroed.
 * Rows past M (or N) only feed C entries that are never stored, so the
 * loaders clamp them to the last row instead of branching.  Offsets are
 * 32-bit from workgroup-uniform bases (the launchers check that they fit). */
template <bool ABF16, int QF = QF_Q8>
__device__ __forceinline__ void gemm_tile(const void* __restrict__ Av, const unsigned char* __restrict__ W,
                                          float* __restrict__ Cm, int M, int N, int K, int lda, int ldc, int tm,
                                          int tn, unsigned short* lds) {
    constexpr unsigned BYTES = QFmt<QF>::BYTES; /* bytes per 32-weight block */
    typedef Stage<ABF16, QF> St;
    constexpr int CPR = ABF16 ? GEMM_BK / 8 : GEMM_BK / 4; /* 16-byte chunks of an A row */
    constexpr int RPP = NTH / CPR;                         /* A rows per loader pass */
    constexpr int NPASS = BM / RPP;
    constexpr int EPC = ABF16 ? 8 : 4;                     /* A elements per chunk */
    const int t = threadIdx.x;
    const int wave = t >> 6, lane = t & 63;
    const int wm = (wave >> 1) * 64, wn = (wave & 1) * 64;
    const int m0 = tm * BM, n0 = tn * BN;
    const int nb = K / 32;                /* blocks of this tile's K range */
    const int nrow = nb;                  /* blocks per weight row */
    const int nfull = nb >> 1;
    const int lr = t >> 1, lh = t & 1;    /* W loader: row, block of the pair */
    const int ar = t / CPR, ac = t % CPR; /* A loader: first row, chunk */
    const float* Af = (const float*)Av + (ABF16 ? 0 : (size_t)m0 * lda);
    const unsigned short* Ah = (const unsigned short*)Av + (ABF16 ? (size_t)m0 * lda : 0);
    const unsigned char* Wb = W + (size_t)n0 * nrow * BYTES;
    unsigned int aoff[NPASS];
#pragma unroll
    for (int p = 0; p < NPASS; p++) aoff[p] = (unsigned)min(ar + RPP * p, M - 1 - m0) * (unsigned)lda + (unsigned)(EPC * ac);
    const unsigned int woff = (unsigned)min(lr, N - 1 - n0) * (unsigned)(nrow * BYTES) + (unsigned)lh * BYTES;

    auto load_a = [&](unsigned int col, St& st) {
#pragma unroll
        for (int p = 0; p < NPASS; p++) {
            if (ABF16)
                __builtin_memcpy(&st.ab[p], __builtin_assume_aligned(Ah + aoff[p] + col, 4), 16);
            else
                __builtin_memcpy(&st.a[p], __builtin_assume_aligned(Af + aoff[p] + col, 4), 16);
        }
    };
    auto load_w = [&](const unsigned char* blk, St& st) {
        __builtin_memcpy(&st.s, __builtin_assume_aligned(blk, 4), 4);
        __builtin_memcpy(&st.q[0], __builtin_assume_aligned(blk + 4, 4), 16);
        if (QF == QF_Q8) __builtin_memcpy(&st.q[QF == QF_Q8 ? 1 : 0], __builtin_assume_aligned(blk + 20, 4), 16);
    };
    auto load = [&](int step, St& st) {
        load_a((unsigned)step * GEMM_BK, st);
        load_w(Wb + woff + (unsigned)step * (2u * BYTES), st);
    };
    /* zero_a: this thread's A chunk lies past K (half step only); the W
     * block past K arrives with scale 0, which zeroes its (finite) q. */
    auto store = [&](int buf, const St& st, bool zero_a) {
        unsigned short* As = lds + buf * 2 * SLAB;
        unsigned short* Bs = As + SLAB;
#pragma unroll
        for (int p = 0; p < NPASS; p++) {
            if (ABF16) {
                *(uint4*)&As[(ar + RPP * p) * LDK + 8 * ac] = zero_a ? make_uint4(0, 0, 0, 0) : st.ab[p];
            } else {
                const float4 v = zero_a ? make_float4(0.f, 0.f, 0.f, 0.f) : st.a[p];
                uint2 u;
                u.x = pk_bf16(v.x, v.y);
                u.y = pk_bf16(v.z, v.w);
                *(uint2*)&As[(ar + RPP * p) * LDK + 4 * ac] = u;
            }
        }
        uint4* bp = (uint4*)&Bs[lr * LDK + 32 * lh];
        if (QF == QF_Q4) {
#pragma unroll
            for (int j = 0; j < 4; j++) bp[j] = dq4(st.q[0], j, st.s);
        } else {
#pragma unroll
            for (int i = 0; i < 2; i++) {
                bp[2 * i] = dq8(st.q[QF == QF_Q8 ? i : 0], 0, st.s);
                bp[2 * i + 1] = dq8(st.q[QF == QF_Q8 ? i : 0], 1, st.s);
            }
        }
    };

    typedef float f32x16 __attribute__((ext_vector_type(16)));
    f32x16 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][j][r] = 0.f;

    const int kq = (lane >> 5) * 8;
    auto mfma_step = [&](int buf) {
        const unsigned short* As = lds + buf * 2 * SLAB;
        const unsigned short* Bs = As + SLAB;
#pragma unroll
        for (int ks = 0; ks < GEMM_BK; ks += 16) {
            bf16x8 fa[2], fb[2];
#pragma unroll
            for (int i = 0; i < 2; i++) fa[i] = *(const bf16x8*)&As[(wm + 32 * i + (lane & 31)) * LDK + ks + kq];
#pragma unroll
            for (int j = 0; j < 2; j++) fb[j] = *(const bf16x8*)&Bs[(wn + 32 * j + (lane & 31)) * LDK + ks + kq];
#pragma unroll
            for (int i = 0; i < 2; i++)
#pragma unroll
                for (int j = 0; j < 2; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[i], fb[j], acc[i][j], 0, 0, 0);
        }
    };

    if (nfull > 0) {
        St s0, s1;
        load(0, s0);
        load(min(1, nfull - 1), s1);
        store(0, s0, false);
        __syncthreads();
        int step = 0;
        /* two steps per iteration so that the register stages are named statically */
        for (; step + 2 <= nfull; step += 2) {
            load(min(step + 2, nfull - 1), s0); /* s0 is free: step's data is in LDS buffer 0 */
            __builtin_amdgcn_sched_barrier(0);  /* keep the loads ahead of the MFMAs */
            mfma_step(0);
            __builtin_amdgcn_sched_barrier(0);
            store(1, s1, false);
            __syncthreads();
            load(min(step + 3, nfull - 1), s1);
            __builtin_amdgcn_sched_barrier(0);
            mfma_step(1);
            __builtin_amdgcn_sched_barrier(0);
            /* unconditional, so that the loads of s0 cannot be sunk next to
             * it; past the end it rewrites buffer 0, which only the half
             * step reuses, after the barrier */
            store(0, s0, false);
            __syncthreads();
        }
        if (step < nfull) mfma_step(0); /* odd step count: the last step sits in buffer 0 */
    }
    if (nb & 1) {
        /* Half step: block nb-1 = 2*nfull.  Buffer (nfull & 1) is free: its
         * last reader was followed by a barrier. */
        St st;
        const int buf = nfull & 1;
        const bool past_a = EPC * ac >= 32; /* this thread's A chunk lies past K */
        load_a(past_a ? 0u : (unsigned)nfull * GEMM_BK, st);
        /* block 2*nfull + 1 (lh = 1) would lie past the row: read block nb-1
         * again and give it scale 0 */
        load_w(Wb + woff + (unsigned)nfull * (2u * BYTES) - (unsigned)lh * BYTES, st);
        if (lh) st.s = 0.0f;
        store(buf, st, past_a);
        __syncthreads();
        mfma_step(buf);
    }

    /* Epilogue, 32x32 D layout: register r of a tile holds row
     * 8*(r/4) + 4*(lane/32) + r%4, column lane%32, so each wave instruction
     * writes 2 rows x 128 bytes: whole 128-byte lines of C when the row
     * pitch is a multiple of 32 floats (measured 2-3% faster than the
     * half-line stores of the 16x16 layout).  Interior tiles store without
     * bounds checks from one base with 32-bit offsets.  C is written once
     * and not read back by this launch, so the stores are nontemporal: they
     * stream past the caches instead of evicting the weight panels that the
     * other M tiles still read (measured 8-10% faster on the 135M prefill
     * set).  Staging the tile through LDS for whole-row stores, and 16-byte
     * stores of a transposed accumulator, both measured slower. */
    float* Ct = Cm + (size_t)(m0 + wm + 4 * (lane >> 5)) * ldc + n0 + wn + (lane & 31);
    if (m0 + BM <= M && n0 + BN <= N) {
#pragma unroll
        for (int i = 0; i < 2; i++)
#pragma unroll
            for (int j = 0; j < 2; j++)
#pragma unroll
                for (int r = 0; r < 16; r++)
                    __builtin_nontemporal_store(acc[i][j][r], &Ct[(unsigned)(32 * i + 8 * (r >> 2) + (r & 3)) * (unsigned)ldc + 32 * j]);
    } else {
#pragma unroll
        for (int i = 0; i < 2; i++)
#pragma unroll
            for (int j = 0; j < 2; j++) {
                const int col = n0 + wn + 32 * j + (lane & 31);
                if (col >= N) continue;
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const int row = m0 + wm + 32 * i + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                    if (row < M) Cm[(size_t)row * ldc + col] = acc[i][j][r];
                }
            }
    }
}

/* Fragment-ordered activations (layout GM_A_FRAG).  A[M][K] in bf16 is
 * stored as 32-row blocks rb and 64-column K steps ks of four 16-deep MFMA
 * A fragments each: fragment (rb, ks, s) is 512 values at
 * ((rb * nks + ks) * 4 + s) * 512, lane l's eight at + 8 l, holding
 * A[32 rb + l % 32][64 ks + 32 (l / 32) + 8 s + j], j < 8; nks = lda / 64
 * (lda: K rounded up to 64), rows past M and columns past K are zero
 * (cast_f32_bf16_frag writes the layout).  The K order inside a step is thus
 * permuted alike in A and W: lane half h of MFMA s takes k = 32 h + 8 s + j,
 * so a wave loads an A fragment with one coalesced 1 KB instruction,
 * straight into registers, and LDS carries the weights only.
 *
 * Tiles of GM_FBM x GM_FBN (256 x 96): 4 waves along M, each 64 x 96 = 2 x 3
 * tiles of v_mfma_f32_32x32x16_bf16.  At M = 512 every weight is
 * dequantised twice (once per 256 rows) and the 96-row weight slab (two
 * buffers) is the whole of LDS; lanes below 192 stage one Q8/Q4 block of it
 * per K step.  Pipeline as gemm_tile: the loads of step s+1 (A) and s+2 (W)
 * are in flight during step s, one barrier per step.  Measured on the 135M
 * M = 512 set against 128 x 128 tiles over row-major bf16: 164-174 us
 * against 207-223 us on the same boxes; the same tiles over row-major A
 * (each wave instruction then touches 32 rows' lines) 210 us, 128 x 128
 * tiles over fragment-ordered A 220 us, 512 x 96 tiles on 8 waves 183 us,
 * 256 x 128 tiles (64 x 128 per wave) 167-171 us. */
constexpr int FB_SLAB = GM_FBN * LDK;

template <int QF>
__device__ __forceinline__ void gemm_tile_frag(const unsigned short* __restrict__ A, const unsigned char* __restrict__ W,
                                               float* __restrict__ Cm, int M, int N, int K, int lda, int ldc, int tm,
                                               int tn, unsigned short* lds) {
    constexpr unsigned BYTES = QFmt<QF>::BYTES;
    const int t = threadIdx.x;
    const int wave = t >> 6, lane = t & 63;
    const int r32 = lane & 31, h = lane >> 5;
    const int m0 = tm * GM_FBM, n0 = tn * GM_FBN;
    const int nb = K / 32, nfull = nb >> 1;
    const int nks = lda / 64, nrb = (M + 31) / 32;
    unsigned int aoff[2];
#pragma unroll
    for (int i = 0; i < 2; i++) {
        const int rb = min((m0 + 64 * wave + 32 * i) / 32, nrb - 1); /* row blocks past M feed no stored C */
        aoff[i] = (unsigned)(rb * nks) * 2048u + 8u * (unsigned)lane;
    }
    const bool wst = t < 2 * GM_FBN; /* W loader lanes: row t/2, block t%2 of the step's pair */
    const int lr = wst ? t >> 1 : 0, lh = t & 1;
    const unsigned int woff = (unsigned)min(n0 + lr, N - 1) * (unsigned)(nb * BYTES) + (unsigned)lh * BYTES;

    struct WSt {
        float s;
        uint4 q[QF == QF_Q4 ? 1 : 2];
    };
    typedef bf16x8 AFr[2][4];
    auto load_a = [&](int step, AFr& fa) {
#pragma unroll
        for (int i = 0; i < 2; i++)
#pragma unroll
            for (int s = 0; s < 4; s++)
                __builtin_memcpy(&fa[i][s], __builtin_assume_aligned(A + aoff[i] + (unsigned)step * 2048u + 512u * s, 16), 16);
    };
    auto load_w = [&](const unsigned char* blk, WSt& w) {
        __builtin_memcpy(&w.s, __builtin_assume_aligned(blk, 4), 4);
        __builtin_memcpy(&w.q[0], __builtin_assume_aligned(blk + 4, 4), 16);
        if (QF == QF_Q8) __builtin_memcpy(&w.q[QF == QF_Q8 ? 1 : 0], __builtin_assume_aligned(blk + 20, 4), 16);
    };
    auto load_wstep = [&](int step, WSt& w) { load_w(W + woff + (unsigned)step * (2u * BYTES), w); };
    auto store_w = [&](int buf, const WSt& w) {
        if (!wst) return;
        uint4* bp = (uint4*)&lds[buf * FB_SLAB + lr * LDK + 32 * lh];
        if (QF == QF_Q4) {
#pragma unroll
            for (int j = 0; j < 4; j++) bp[j] = dq4(w.q[0], j, w.s);
        } else {
#pragma unroll
            for (int i = 0; i < 2; i++) {
                bp[2 * i] = dq8(w.q[QF == QF_Q8 ? i : 0], 0, w.s);
                bp[2 * i + 1] = dq8(w.q[QF == QF_Q8 ? i : 0], 1, w.s);
            }
        }
    };

    typedef float f32x16 __attribute__((ext_vector_type(16)));
    f32x16 acc[2][3];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 3; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][j][r] = 0.f;

    auto mfma_step = [&](int buf, const AFr& fa) {
        const unsigned short* Bs = lds + buf * FB_SLAB;
#pragma unroll
        for (int s = 0; s < 4; s++) {
            bf16x8 fb[3];
#pragma unroll
            for (int j = 0; j < 3; j++) fb[j] = *(const bf16x8*)&Bs[(32 * j + r32) * LDK + 32 * h + 8 * s];
#pragma unroll
            for (int i = 0; i < 2; i++)
#pragma unroll
                for (int j = 0; j < 3; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[i][s], fb[j], acc[i][j], 0, 0, 0);
        }
    };

    if (nfull > 0) {
        AFr fa0, fa1;
        WSt w0, w1;
        load_wstep(0, w0);
        load_a(0, fa0);
        load_wstep(min(1, nfull - 1), w1);
        store_w(0, w0);
        __syncthreads();
        int step = 0;
        /* two steps per iteration so that the register stages are named
         * statically; past the last step the loads repeat it (cache hits,
         * never used) */
        for (; step + 2 <= nfull; step += 2) {
            load_a(min(step + 1, nfull - 1), fa1);
            load_wstep(min(step + 2, nfull - 1), w0);
            __builtin_amdgcn_sched_barrier(0); /* keep the loads ahead of the MFMAs */
            mfma_step(0, fa0);
            __builtin_amdgcn_sched_barrier(0);
            store_w(1, w1);
            __syncthreads();
            load_a(min(step + 2, nfull - 1), fa0);
            load_wstep(min(step + 3, nfull - 1), w1);
            __builtin_amdgcn_sched_barrier(0);
            mfma_step(1, fa1);
            __builtin_amdgcn_sched_barrier(0);
            store_w(0, w0);
            __syncthreads();
        }
        if (step < nfull) mfma_step(0, fa0); /* odd step count: the last step sits in buffer 0 */
    }
    if (nb & 1) {
        /* half step (block nb-1 = 2*nfull): A's columns past K are zero in
         * the layout; block 2*nfull + 1 would lie past the row, so lh = 1
         * reads block nb-1 again with scale 0 (which zeroes its finite
         * codes).  Buffer nfull & 1 is free: its last reader was followed by
         * a barrier. */
        AFr fa;
        WSt w;
        const int buf = nfull & 1;
        load_a(nfull, fa);
        load_w(W + woff + (unsigned)nfull * (2u * BYTES) - (unsigned)lh * BYTES, w);
        if (lh) w.s = 0.0f;
        store_w(buf, w);
        __syncthreads();
        mfma_step(buf, fa);
    }

    /* epilogue, 32x32 D layout as in gemm_tile: whole 128-byte C row lines,
     * nontemporal stores for interior tiles */
    float* Ct = Cm + (size_t)(m0 + 64 * wave + 4 * h) * ldc + n0 + r32;
    if (m0 + GM_FBM <= M && n0 + GM_FBN <= N) {
#pragma unroll
        for (int i = 0; i < 2; i++)
#pragma unroll
            for (int j = 0; j < 3; j++)
#pragma unroll
                for (int r = 0; r < 16; r++)
                    __builtin_nontemporal_store(acc[i][j][r], &Ct[(unsigned)(32 * i + 8 * (r >> 2) + (r & 3)) * (unsigned)ldc + 32 * j]);
    } else {
#pragma unroll
        for (int i = 0; i < 2; i++)
#pragma unroll
            for (int j = 0; j < 3; j++) {
                const int col = n0 + 32 * j + r32;
                if (col >= N) continue;
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const int row = m0 + 64 * wave + 32 * i + 8 * (r >> 2) + 4 * h + (r & 3);
                    if (row < M) Cm[(size_t)row * ldc + col] = acc[i][j][r];
                }
            }
    }
}

template <int QF>
__global__ __launch_bounds__(NTH) __attribute__((amdgpu_waves_per_eu(2, 2))) void k_gemm_multi_frag(
    const void* __restrict__ A, const unsigned char* __restrict__ W, float* __restrict__ C,
    const GmDesc* __restrict__ desc, const unsigned int* __restrict__ tile_map) {
    __shared__ __attribute__((aligned(16))) unsigned short lds[2 * FB_SLAB];
    const unsigned int tm_ = tile_map[blockIdx.x];
    if (tm_ == GM_IDLE_TILE) return;
    const GmDesc d = desc[tm_ >> 16];
    const int tile = (int)(tm_ & 0xffffu);
    const int tiles_n = (d.N + GM_FBN - 1) / GM_FBN;
    gemm_tile_frag<QF>((const unsigned short*)A + d.a_off, W + d.w_off, C + d.c_off, d.M, d.N, d.K, d.lda, d.ldc,
                       tile / tiles_n, tile % tiles_n, lds);
}

/* fp32 [M][lda] -> bf16 in fragment order (see gemm_tile_frag), round to
 * nearest even; one 16-byte fragment slot (8 values) per lane. */
__global__ __launch_bounds__(NTH) void k_cast_bf16_frag(const float* __restrict__ src, unsigned short* __restrict__ dst,
                                                        int M, int K, int lda, int nks, long nslots) {
    const long i = (long)blockIdx.x * NTH + threadIdx.x;
    if (i >= nslots) return;
    const int lane = (int)(i & 63), s = (int)((i >> 6) & 3);
    const long rk = i >> 8;
    const int ks = (int)(rk % nks), rb = (int)(rk / nks);
    const int row = 32 * rb + (lane & 31), col = 64 * ks + 32 * (lane >> 5) + 8 * s;
    uint4 v = make_uint4(0u, 0u, 0u, 0u);
    if (row < M && col < K) { /* K is a multiple of 32: the slot's 8 columns are all inside */
        float4 a, b;
        const float* sp = src + (size_t)row * lda + col;
        __builtin_memcpy(&a, __builtin_assume_aligned(sp, 4), 16);
        __builtin_memcpy(&b, __builtin_assume_aligned(sp + 4, 4), 16);
        v.x = pk_bf16(a.x, a.y);
        v.y = pk_bf16(a.z, a.w);
        v.z = pk_bf16(b.x, b.y);
        v.w = pk_bf16(b.z, b.w);
    }
    __builtin_memcpy(dst + 8 * i, &v, 16);
}

template <int QF>
__device__ __forceinline__ void gemm_group_body(const GmGroup& g, unsigned short* lds) {
    int tile = blockIdx.x;
    int pi = 0;
    while (pi + 1 < g.nprob && tile >= g.p[pi].tiles) {
        tile -= g.p[pi].tiles;
        pi++;
    }
    const GmProb& p = g.p[pi];
    const int tiles_n = (p.N + BN - 1) / BN;
    gemm_tile<false, QF>(p.A, p.W, p.C, p.M, p.N, p.K, p.lda, p.ldc, tile / tiles_n, tile % tiles_n, lds);
}

__global__ __launch_bounds__(NTH) __attribute__((amdgpu_waves_per_eu(2, 2))) void k_q8_gemm(GmGroup g) {
    __shared__ __attribute__((aligned(16))) unsigned short lds[GEMM_LDS];
    gemm_group_body<QF_Q8>(g, lds);
}

/* The same over Q4_0 weights (reference forward.metal:829-858 at BT > 1). */
__global__ __launch_bounds__(NTH) __attribute__((amdgpu_waves_per_eu(2, 2))) void k_q4_gemm(GmGroup g) {
    __shared__ __attribute__((aligned(16))) unsigned short lds[GEMM_LDS];
    gemm_group_body<QF_Q4>(g, lds);
}

template <bool ABF16, int QF>
__device__ __forceinline__ void gemm_multi_body(const void* __restrict__ A, const unsigned char* __restrict__ W,
                                                float* __restrict__ C, const GmDesc* __restrict__ desc,
                                                const unsigned int* __restrict__ tile_map, unsigned short* lds) {
    const unsigned int tm_ = tile_map[blockIdx.x];
    if (tm_ == GM_IDLE_TILE) return;
    const GmDesc d = desc[tm_ >> 16];
    const int tile = (int)(tm_ & 0xffffu);
    const int tiles_n = (d.N + BN - 1) / BN;
    const void* Ad = ABF16 ? (const void*)((const unsigned short*)A + d.a_off) : (const void*)((const float*)A + d.a_off);
    gemm_tile<ABF16, QF>(Ad, W + d.w_off, C + d.c_off, d.M, d.N, d.K, d.lda, d.ldc, tile / tiles_n, tile % tiles_n, lds);
}

/* Activations in fp32 (cast to bf16 while staging) or already in bf16. */
template <bool ABF16>
__global__ __launch_bounds__(NTH) __attribute__((amdgpu_waves_per_eu(2, 2))) void k_q8_gemm_multi(const void* __restrict__ A, const unsigned char* __restrict__ W,
                                                       float* __restrict__ C, const GmDesc* __restrict__ desc,
                                                       const unsigned int* __restrict__ tile_map) {
    __shared__ __attribute__((aligned(16))) unsigned short lds[GEMM_LDS];
    gemm_multi_body<ABF16, QF_Q8>(A, W, C, desc, tile_map, lds);
}

template <bool ABF16>
__global__ __launch_bounds__(NTH) __attribute__((amdgpu_waves_per_eu(2, 2))) void k_q4_gemm_multi(const void* __restrict__ A, const unsigned char* __restrict__ W,
                                                       float* __restrict__ C, const GmDesc* __restrict__ desc,
                                                       const unsigned int* __restrict__ tile_map) {
    __shared__ __attribute__((aligned(16))) unsigned short lds[GEMM_LDS];
    gemm_multi_body<ABF16, QF_Q4>(A, W, C, desc, tile_map, lds);
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
extern "C" int gm_tiles_frag(int M, int N) { return ((M + GM_FBM - 1) / GM_FBM) * ((N + GM_FBN - 1) / GM_FBN); }

/* The tile loaders address a problem with 32-bit offsets. */
static bool gm_offsets_fit(int M, int N, int K, int lda) {
    return (unsigned long long)M * (unsigned long long)lda < 0x80000000ull &&
           (unsigned long long)N * (unsigned long long)(K / 32) * 36ull < 0x80000000ull;
}

static bool gm_offsets_fit_q(int M, int N, int K, int lda, unsigned bytes) {
    return (unsigned long long)M * (unsigned long long)lda < 0x80000000ull &&
           (unsigned long long)N * (unsigned long long)(K / 32) * bytes < 0x80000000ull;
}

/* The group launch over Q4_0 weights (qf 1) or Q8_0 (qf 0). */
extern "C" int gm_launch_group_qf(GmGroup* g, int qf, hipStream_t s) {
    if (qf == 0) return gm_launch_group(g, s);
    long total = 0;
    for (int i = 0; i < g->nprob; i++)
        BMK_REQUIRE(gm_offsets_fit_q(g->p[i].M, g->p[i].N, g->p[i].K, g->p[i].lda, 20u),
                    "q4 gemm: problem %d too large for 32-bit tile offsets", i);
    for (int i = 0; i < g->nprob; i++) {
        g->p[i].tiles = gm_tiles_for(g->p[i].M, g->p[i].N);
        total += g->p[i].tiles;
    }
    if (total <= 0) return 0;
    hipLaunchKernelGGL(k_q4_gemm, dim3((unsigned)total), dim3(NTH), 0, s, *g);
    BMK_LAUNCH_CHECK();
    return 0;
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
template <int QF>
static int launch_gemm_multi(const bmk_launch_t* a) {
    constexpr unsigned BYTES = QFmt<QF>::BYTES;
    BMK_NEED_BYTES(a, 0, 8, "params");
    const int nprob = bmk_pi(a, 0, 0), n_tiles = bmk_pi(a, 0, 1);
    const int layout = a->bytes[0] >= 12 ? bmk_pi(a, 0, 2) : GM_A_F32;
    const int a_bf16 = layout != GM_A_F32;
    const bool frag = layout == GM_A_FRAG;
    const unsigned long long esz = a_bf16 ? 2 : 4; /* bytes per activation element */
    BMK_REQUIRE(nprob >= 0 && n_tiles >= 0 && layout >= GM_A_F32 && layout <= GM_A_FRAG,
                "q8 gemm multi: bad params nprob=%d n_tiles=%d layout=%d", nprob, n_tiles, layout);
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
        BMK_REQUIRE(d.pad_ == 0, "q8 gemm multi: problem %d has a nonzero reserved field", i);
        const int want_tiles = frag ? gm_tiles_frag(d.M, d.N) : gm_tiles_for(d.M, d.N);
        BMK_REQUIRE(d.tiles == want_tiles && d.tile0 == next_tile,
                    "q8 gemm multi: problem %d tiles %d@%d, expected %d@%ld", i, d.tiles, d.tile0, want_tiles,
                    next_tile);
        BMK_REQUIRE((d.w_off & 3) == 0, "q8 gemm multi: problem %d weight offset not 4-byte aligned", i);
        BMK_REQUIRE(gm_offsets_fit_q(d.M, d.N, d.K, d.lda, BYTES),
                    "q8 gemm multi: problem %d too large for 32-bit tile offsets", i);
        BMK_REQUIRE((!a_bf16 || (d.a_off % 8 == 0 && d.lda % 8 == 0)),
                    "q8 gemm multi: problem %d bf16 rows must start 16-byte aligned", i);
        /* fragment order: lda = K rounded up to 64, ceil(M/32) blocks of 32 rows, 1 KB-aligned fragments */
        const unsigned long long a_end = frag ? d.a_off + (unsigned long long)((d.M + 31) / 32) * 32ull * d.lda
                                              : d.a_off + (unsigned long long)(d.M - 1) * d.lda + d.K;
        BMK_REQUIRE(!frag || (d.lda % 64 == 0 && d.lda < d.K + 64 && d.a_off % 512 == 0 &&
                              (unsigned long long)((d.M + 31) / 32) * 32ull * d.lda < 0x80000000ull),
                    "q8 gemm multi: problem %d fragment-order activations need lda = K rounded up to 64 and "
                    "a 512-element-aligned offset (lda=%d K=%d a_off=%llu)", i, d.lda, d.K, d.a_off);
        BMK_REQUIRE(a_end <= a->bytes[2] / esz &&
                        d.w_off + (unsigned long long)d.N * (d.K / 32) * BYTES <= a->bytes[3] &&
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
    if (a_bf16) BMK_REQUIRE(((uintptr_t)a->dev[2] & 15) == 0, "q8 gemm multi: bf16 activation arena must be 16-byte aligned");
    const dim3 grid((unsigned)n_tiles), tb(NTH);
    const void* A = (const void*)a->dev[2];
    const unsigned char* W = (const unsigned char*)a->dev[3];
    float* C = (float*)a->dev[4];
    if (frag) {
        hipLaunchKernelGGL(k_gemm_multi_frag<QF>, grid, tb, 0, a->stream, A, W, C, dd, dt);
    } else if (QF == QF_Q4) {
        if (a_bf16) hipLaunchKernelGGL(k_q4_gemm_multi<true>, grid, tb, 0, a->stream, A, W, C, dd, dt);
        else hipLaunchKernelGGL(k_q4_gemm_multi<false>, grid, tb, 0, a->stream, A, W, C, dd, dt);
    } else {
        if (a_bf16) hipLaunchKernelGGL(k_q8_gemm_multi<true>, grid, tb, 0, a->stream, A, W, C, dd, dt);
        else hipLaunchKernelGGL(k_q8_gemm_multi<false>, grid, tb, 0, a->stream, A, W, C, dd, dt);
    }
    BMK_LAUNCH_CHECK();
    return 0;
}

extern "C" int bmk_launch_q8_gemm_multi(const bmk_launch_t* a) { return launch_gemm_multi<QF_Q8>(a); }
extern "C" int bmk_launch_q4_gemm_multi(const bmk_launch_t* a) { return launch_gemm_multi<QF_Q4>(a); }

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

/* cast_f32_bf16_frag {src f32 [M][lda], dst bf16 in fragment order, params int{M, K, lda}}:
 * the activations of a matmul_forward_q8_multi problem with layout 2 (the
 * destination holds ceil(M/32) x ceil(K/64) x 2048 values, padding zeroed;
 * the problem's lda is K rounded up to 64). */
extern "C" int gm_cast_bf16_frag(const float* src, unsigned short* dst, int M, int K, int lda, hipStream_t s) {
    BMK_REQUIRE(M > 0 && K > 0 && K % 32 == 0 && lda >= K, "cast_f32_bf16_frag: bad params M=%d K=%d lda=%d", M, K,
                lda);
    const long nrb = (M + 31) / 32, nks = (K + 63) / 64;
    const long nslots = nrb * nks * 256; /* 16-byte slots: 4 fragments x 64 lanes per (block, step) */
    BMK_REQUIRE(nrb * 32 * nks * 64 < 0x80000000L, "cast_f32_bf16_frag: %d x %d is too large", M, K);
    BMK_REQUIRE(((uintptr_t)src & 3) == 0 && ((uintptr_t)dst & 15) == 0,
                "cast_f32_bf16_frag: src must be 4-byte and dst 16-byte aligned");
    hipLaunchKernelGGL(k_cast_bf16_frag, dim3((unsigned)((nslots + NTH - 1) / NTH)), dim3(NTH), 0, s, src, dst, M, K,
                       lda, (int)nks, nslots);
    BMK_LAUNCH_CHECK();
    return 0;
}

extern "C" int bmk_launch_cast_bf16_frag(const bmk_launch_t* a) {
    BMK_NEED_BYTES(a, 2, 12, "params");
    const int M = bmk_pi(a, 2, 0), K = bmk_pi(a, 2, 1), lda = bmk_pi(a, 2, 2);
    BMK_REQUIRE(M > 0 && K > 0 && K % 32 == 0 && lda >= K, "cast_f32_bf16_frag: bad params M=%d K=%d lda=%d", M, K,
                lda);
    BMK_NEED_BYTES(a, 0, ((size_t)(M - 1) * lda + K) * 4, "src");
    BMK_NEED_BYTES(a, 1, (size_t)((M + 31) / 32) * ((K + 63) / 64) * 256 * 16, "dst");
    return gm_cast_bf16_frag((const float*)a->dev[0], (unsigned short*)a->dev[1], M, K, lda, a->stream);
}

/* Multi-GEMM launch from a device-resident plan built by bm_q8_gemm_plan
 * (the engine's prefill; the plan was validated when it was built); qf 1:
 * Q4_0 weights. */
extern "C" int gm_launch_multi_qf(const void* A, int a_bf16, int qf, const unsigned char* W, float* C, const void* plan,
                                  int nprob, int n_tiles, hipStream_t s) {
    if (nprob <= 0 || n_tiles <= 0) return 0;
    const GmDesc* desc = (const GmDesc*)plan;
    const unsigned int* tmap = (const unsigned int*)((const char*)plan + (size_t)nprob * sizeof(GmDesc));
    const dim3 grid((unsigned)n_tiles), tb(NTH);
    if (qf) {
        if (a_bf16) hipLaunchKernelGGL(k_q4_gemm_multi<true>, grid, tb, 0, s, A, W, C, desc, tmap);
        else hipLaunchKernelGGL(k_q4_gemm_multi<false>, grid, tb, 0, s, A, W, C, desc, tmap);
    } else {
        if (a_bf16) hipLaunchKernelGGL(k_q8_gemm_multi<true>, grid, tb, 0, s, A, W, C, desc, tmap);
        else hipLaunchKernelGGL(k_q8_gemm_multi<false>, grid, tb, 0, s, A, W, C, desc, tmap);
    }
    BMK_LAUNCH_CHECK();
    return 0;
}

extern "C" int gm_launch_multi(const void* A, int a_bf16, const unsigned char* W, float* C, const void* plan, int nprob,
                               int n_tiles, hipStream_t s) {
    return gm_launch_multi_qf(A, a_bf16, 0, W, C, plan, nprob, n_tiles, s);
}

/* fp32 -> bf16 over n elements (RNE) */
extern "C" int gm_cast_bf16(const float* src, unsigned short* dst, long n, hipStream_t s) {
    if (n <= 0) return 0;
    const long n8 = n / 8;
    hipLaunchKernelGGL(k_cast_bf16, dim3((unsigned)((n8 + NTH) / NTH)), dim3(NTH), 0, s, src, dst, n8, n);
    BMK_LAUNCH_CHECK();
    return 0;
}
