/* SPDX-License-Identifier: MPL-2.0
 *
 * pf_gemm.hip — the per-layer projections of the engine's prefill
 * (reference session.c:86-139, which runs them as matmul_forward_q8,
 * forward.metal:625-649, then separate residual and SwiGLU kernels):
 *
 *   C[m][n] = sum_k A[m][k] * bf16(q[n][k] * scale[n][k/32])   (A bf16, fp32 accumulation)
 *
 * with the same operand roundings as q8_gemm.hip.  At a prompt of a few
 * hundred tokens a layer's projection has tens to a few hundred 32x64 or
 * 64x64 output tiles: each launch runs about one tile per CU, and its time
 * is one tile's dependent chain (loads, dequantisation, MFMAs, stores), not
 * the chip's throughput.  The kernel keeps that chain short:
 *  - no LDS staging and no barrier in the K loop.  Lane l of a wave (MFMA
 *    column l % 32, half h = l / 32) owns one whole 32-wide K block per
 *    64-wide step s, block 2s + h, of its two A rows and its two weight
 *    rows; MFMA u (0..3) of the step takes the lane's values 8u .. 8u+7 of
 *    that block on both sides, so the contraction runs over
 *    k = 64s + 32h + 8u + j in A and W alike.  Both operands are stored in
 *    that order, so every load instruction of a wave reads one contiguous
 *    span, straight into registers: the activations in MFMA fragment order
 *    (written so by their producers: the RMSNorm, the attention, the SwiGLU
 *    epilogue), the weights in the prefill layout (pf_gemm.h, a copy the
 *    engine makes once per model).  Scattered 16-byte loads (32 rows per
 *    instruction) cost 2.7-4.8 us more per launch at 512 tokens;
 *  - the four waves of a workgroup split K (contiguous step ranges), with
 *    the loads of three steps in flight, and sum their partial tiles through
 *    LDS once at the end, in wave order (the same bits every run);
 *  - the consumer runs in the epilogue: the plain store, the q/k/v
 *    epilogue (k rotated by RoPE and appended to the KV cache with v, as
 *    the reference's rope and cache-append kernels do, forward.metal:1284-
 *    1329), the residual add (o, down: x += C, one writer per element), or
 *    SwiGLU (gate and up rows of the same outputs in one tile, bf16 out for
 *    the down projection), so no partial copies of C are written or re-read.
 */
#include "bmk.h"
#include "pf_gemm.h"
#include "q8_common.h"

namespace {

using bmk::QFmt;
using bmk::QF_Q8;
using bmk::QF_Q4;
using bmk::q4_code;
using bmk::frag_index;
using bmk::silu_mul;

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

constexpr int PT = PFG_TILE;
constexpr int PLD = PT + 4; /* LDS row of a partial tile, floats */
constexpr int PNTH = 256;   /* 4 waves */

__device__ __forceinline__ unsigned int pk2(float lo, float hi) {
    const f32x2 v = {lo, hi};
    const bf16x2 r = __builtin_convertvector(v, bf16x2);
    unsigned int u;
    __builtin_memcpy(&u, &r, 4);
    return u;
}

__device__ __forceinline__ float sb(unsigned int w, int k) { return (float)(signed char)((w >> (8 * k)) & 0xffu); }

/* One lane's operands of one 64-wide K step: its A block in both row
 * groups (32 bf16 each) and its weight block in both column groups. */
template <int QF, int MI, int NJ>
struct PfgStage {
    uint4 a[MI][4];
    float s[NJ];
    uint4 q[NJ][QF == QF_Q4 ? 1 : 2];
};

/* Codes 8u .. 8u+7 of a block, times its scale, rounded to bf16. */
template <int QF>
__device__ __forceinline__ bf16x8 dq(const uint4* q, int u, float s) {
    unsigned int w0, w1;
    uint4 r;
    if (QF == QF_Q4) {
        const unsigned int w = u == 0 ? q[0].x : u == 1 ? q[0].y : u == 2 ? q[0].z : q[0].w;
        r.x = pk2(q4_code(w, 0) * s, q4_code(w, 1) * s);
        r.y = pk2(q4_code(w, 2) * s, q4_code(w, 3) * s);
        r.z = pk2(q4_code(w, 4) * s, q4_code(w, 5) * s);
        r.w = pk2(q4_code(w, 6) * s, q4_code(w, 7) * s);
    } else {
        const uint4& h = q[u >> 1];
        w0 = (u & 1) ? h.z : h.x;
        w1 = (u & 1) ? h.w : h.y;
        r.x = pk2(sb(w0, 0) * s, sb(w0, 1) * s);
        r.y = pk2(sb(w0, 2) * s, sb(w0, 3) * s);
        r.z = pk2(sb(w1, 0) * s, sb(w1, 1) * s);
        r.w = pk2(sb(w1, 2) * s, sb(w1, 3) * s);
    }
    bf16x8 b;
    __builtin_memcpy(&b, &r, 16);
    return b;
}

template <int QF, int EPI, int MI, int NJ>
__global__ __launch_bounds__(PNTH) void k_pf_gemm(PfgArgs a) {
    constexpr int PTM = 32 * MI;  /* tile rows */
    constexpr int TW = 32 * NJ;   /* tile columns */
    constexpr int CPT = 8 * NJ;   /* epilogue columns per thread */
    static_assert(NJ == 2 || EPI == PFG_RESID || EPI == PFG_STORE, "gate/up pairs and RoPE pairs need 64 columns");
    __shared__ float part[4][PTM][TW + 4];
    __shared__ float sst[PFG_SS_MAX][PT]; /* the tile rows' partial sums of squares */
    constexpr unsigned CH = QF == QF_Q4 ? PFG_CHUNK_Q4 : PFG_CHUNK_Q8;
    const int t = threadIdx.x, wave = t >> 6, lane = t & 63;
    const int col = lane & 31, h = lane >> 5;
    const int nt = (int)(blockIdx.x % (unsigned)a.NT), mt = (int)(blockIdx.x / (unsigned)a.NT);
    const int M = a.M, ns = (a.K + 63) >> 6; /* 64-wide K steps (fragment columns per row block) */
    const int m0 = mt * PTM;
    int p = 0;
    if (EPI != PFG_SWIGLU) {
        if (a.nprob > 1 && nt >= a.p[1].tile0) p = 1;
        if (a.nprob > 2 && nt >= a.p[2].tile0) p = 2;
    }
    const int N = a.p[p].N, nfr = (N + 31) >> 5;
    /* SwiGLU: column group 0 holds gate rows n0 .. n0+31, group 1 the up
     * rows of the same outputs */
    const int n0 = EPI == PFG_SWIGLU ? nt * 32 : (nt - a.p[p].tile0) * TW;
    /* Rows past M (N) only feed C entries that are never stored: the row
     * blocks (chunks) past the last are clamped to it. */
    const unsigned short* af[MI];
    const unsigned char* wc[NJ];
#pragma unroll
    for (int i = 0; i < MI; i++) {
        const int rb = min((m0 >> 5) + i, ((M + 31) >> 5) - 1);
        af[i] = a.A + (size_t)rb * ns * 2048 + 8 * lane;
    }
#pragma unroll
    for (int i = 0; i < NJ; i++) {
        const int f = min(EPI == PFG_SWIGLU ? nt : (n0 >> 5) + i, nfr - 1);
        wc[i] = a.W + a.p[EPI == PFG_SWIGLU ? i : p].w_off + (size_t)f * ns * CH;
    }
    const int s_beg = wave * ns / 4, s_end = (wave + 1) * ns / 4;
    /* Epilogue thread map: row r of the tile; CPT columns from c0 (8 gate
     * and 8 up columns from j0 for SwiGLU). */
    const int r = t >> 2, m = m0 + r, c0 = (t & 3) * CPT, j0 = (t & 3) * 8;
    const int ldc = a.p[p].ldc;
    float* dst = EPI == PFG_RESID ? a.x + (size_t)min(m, M - 1) * ldc + n0 + c0
                                  : (EPI == PFG_STORE || (EPI == PFG_QKV && p == 0)
                                         ? a.p[p].C + (size_t)min(m, M - 1) * ldc + n0 + c0
                                         : nullptr);
    const bool whole = (EPI == PFG_STORE || EPI == PFG_RESID || (EPI == PFG_QKV && p == 0)) && n0 + c0 + CPT <= N &&
                       ((uintptr_t)dst & 15) == 0;
    /* the residual rows this thread adds to, loaded before the K loop so
     * that their latency hides behind it */
    float4 res[CPT / 4];
    if (EPI == PFG_RESID && whole && r < PTM) {
#pragma unroll
        for (int c = 0; c < CPT / 4; c++) res[c] = *(const float4*)&dst[4 * c];
    }
    /* The RMSNorm inputs, loaded before the K loop so that their latency
     * hides behind it: the tile rows' partial sums of squares, straight
     * into LDS (global_load_lds: one tile's 64 rows per wave instruction,
     * no registers held across the loop), or, for a residual launch that
     * writes the next norm's operand, the norm weights of its 16 columns. */
    if (EPI != PFG_RESID && a.ss_in) {
        for (int i = wave; i < a.ss_tiles; i += 4)
            __builtin_amdgcn_global_load_lds(
                (const __attribute__((address_space(1))) void*)(a.ss_in + (size_t)i * a.ss_ld + min(m0 + lane, M - 1)),
                (__attribute__((address_space(3))) void*)&sst[i][0], 4, 0, 0);
    }
    float gnr[CPT];
    if (EPI == PFG_RESID && a.an && r < PTM) {
#pragma unroll
        for (int c = 0; c < CPT; c++) gnr[c] = a.gn[min(n0 + c0 + c, N - 1)];
    }

    auto load = [&](int s, PfgStage<QF, MI, NJ>& st) {
#pragma unroll
        for (int i = 0; i < MI; i++)
#pragma unroll
            for (int u = 0; u < 4; u++)
                __builtin_memcpy(&st.a[i][u], __builtin_assume_aligned(af[i] + (size_t)s * 2048 + 512 * u, 16), 16);
#pragma unroll
        for (int j = 0; j < NJ; j++) {
            const unsigned char* c = wc[j] + (size_t)s * CH;
            __builtin_memcpy(&st.s[j], __builtin_assume_aligned(c + 4 * lane, 4), 4);
            __builtin_memcpy(&st.q[j][0], __builtin_assume_aligned(c + 256 + 16 * lane, 16), 16);
            if (QF == QF_Q8) __builtin_memcpy(&st.q[j][QF == QF_Q8 ? 1 : 0], __builtin_assume_aligned(c + 1280 + 16 * lane, 16), 16);
        }
    };

    f32x16 acc[MI][NJ];
#pragma unroll
    for (int i = 0; i < MI; i++)
#pragma unroll
        for (int j = 0; j < NJ; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][j][r] = 0.f;

    /* Past an odd block count the last step's upper half is zero on both
     * sides (the producers' column padding, the layout's zero blocks). */
    auto compute = [&](const PfgStage<QF, MI, NJ>& st) {
#pragma unroll
        for (int u = 0; u < 4; u++) {
            bf16x8 fb[NJ], fa[MI];
#pragma unroll
            for (int j = 0; j < NJ; j++) fb[j] = dq<QF>(st.q[j], u, st.s[j]);
#pragma unroll
            for (int i = 0; i < MI; i++) __builtin_memcpy(&fa[i], &st.a[i][u], 16);
#pragma unroll
            for (int i = 0; i < MI; i++)
#pragma unroll
                for (int j = 0; j < NJ; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[i], fb[j], acc[i][j], 0, 0, 0);
        }
    };

    /* Groups of three steps: all loads of a group are issued first (past
     * the wave's last step they repeat it: an L2 hit, never used, so every
     * path issues the same loads), then each step waits for its own. */
    for (int g = s_beg; g < s_end; g += 3) {
        PfgStage<QF, MI, NJ> s0, s1, s2;
        load(g, s0);
        load(min(g + 1, s_end - 1), s1);
        load(min(g + 2, s_end - 1), s2);
        __builtin_amdgcn_sched_barrier(0);
        compute(s0);
        if (g + 1 < s_end) compute(s1);
        if (g + 2 < s_end) compute(s2);
    }

    /* Partial tiles to LDS (32x32 D layout: register r of a tile holds row
     * 8 (r / 4) + 4 h + r % 4, column l % 32), then the sum in wave order. */
#pragma unroll
    for (int i = 0; i < MI; i++)
#pragma unroll
        for (int j = 0; j < NJ; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) part[wave][32 * i + 8 * (r >> 2) + 4 * h + (r & 3)][32 * j + col] = acc[i][j][r];
    if (EPI != PFG_RESID && a.ss_in) asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); /* the sums have landed */
    __syncthreads();
    if (r >= PTM || m >= M) return; /* the epilogue's map: four threads per tile row */
    float inv = 1.0f;
    if (EPI != PFG_RESID && a.ss_in) {
        float ss = 0.f;
        for (int i = 0; i < a.ss_tiles; i++) ss += sst[i][r]; /* tile order */
        inv = 1.0f / sqrtf(ss / (float)a.norm_d + a.eps);
    }
    /* C is written once and read by the next kernel: the stores stream
     * (nontemporal), leaving less for the end of the launch to write back */
    if (EPI == PFG_SWIGLU) {
        float g[8], u[8];
#pragma unroll
        for (int c = 0; c < 8; c += 4) {
            float4 gv = *(const float4*)&part[0][r][j0 + c], uv = *(const float4*)&part[0][r][32 + j0 + c];
#pragma unroll
            for (int w = 1; w < 4; w++) {
                const float4 gw = *(const float4*)&part[w][r][j0 + c], uw = *(const float4*)&part[w][r][32 + j0 + c];
                gv.x += gw.x; gv.y += gw.y; gv.z += gw.z; gv.w += gw.w;
                uv.x += uw.x; uv.y += uw.y; uv.z += uw.z; uv.w += uw.w;
            }
            g[c] = gv.x * inv; g[c + 1] = gv.y * inv; g[c + 2] = gv.z * inv; g[c + 3] = gv.w * inv;
            u[c] = uv.x * inv; u[c + 1] = uv.y * inv; u[c + 2] = uv.z * inv; u[c + 3] = uv.w * inv;
        }
        /* eight consecutive columns: eight consecutive values of the
         * fragment-ordered output; columns past N (up to the next multiple
         * of 64) are the down projection's zero padding */
        uint4 o = make_uint4(0u, 0u, 0u, 0u);
        unsigned int* ov = &o.x;
#pragma unroll
        for (int c = 0; c < 8; c += 2) {
            const float lo = n0 + j0 + c < N ? silu_mul(g[c], u[c]) : 0.f;
            const float hi = n0 + j0 + c + 1 < N ? silu_mul(g[c + 1], u[c + 1]) : 0.f;
            ov[c >> 1] = pk2(lo, hi);
        }
        const u32x4 ov4 = {o.x, o.y, o.z, o.w};
        __builtin_nontemporal_store(ov4, (u32x4*)(a.h + frag_index(m, n0 + j0, (N + 63) >> 6)));
    } else if (EPI == PFG_QKV && p == 2) {
        /* a tile is one KV head (64 columns): v rows into the V cache */
        float* vr = a.vc + (size_t)m * N + n0 + c0;
#pragma unroll
        for (int c = 0; c < 16; c += 4) {
            float4 v4 = *(const float4*)&part[0][r][c0 + c];
#pragma unroll
            for (int w = 1; w < 4; w++) {
                const float4 pw = *(const float4*)&part[w][r][c0 + c];
                v4.x += pw.x; v4.y += pw.y; v4.z += pw.z; v4.w += pw.w;
            }
            *(float4*)&vr[c] = make_float4(v4.x * inv, v4.y * inv, v4.z * inv, v4.w * inv);
        }
    } else if (EPI == PFG_QKV) {
        /* q and k: RoPE pairs (d, d + 32) of the tile's head, eight per
         * thread (d from j0), with the position's cos / sin from the table;
         * rotated q rows go to q, k rows to the K cache, [dim / 4][position][4] */
        float k0[8], k1[8];
#pragma unroll
        for (int c = 0; c < 8; c += 4) {
            float4 lo = *(const float4*)&part[0][r][j0 + c], hi = *(const float4*)&part[0][r][32 + j0 + c];
#pragma unroll
            for (int w = 1; w < 4; w++) {
                const float4 lw = *(const float4*)&part[w][r][j0 + c], hw = *(const float4*)&part[w][r][32 + j0 + c];
                lo.x += lw.x; lo.y += lw.y; lo.z += lw.z; lo.w += lw.w;
                hi.x += hw.x; hi.y += hw.y; hi.z += hw.z; hi.w += hw.w;
            }
            k0[c] = lo.x * inv; k0[c + 1] = lo.y * inv; k0[c + 2] = lo.z * inv; k0[c + 3] = lo.w * inv;
            k1[c] = hi.x * inv; k1[c + 1] = hi.y * inv; k1[c + 2] = hi.z * inv; k1[c + 3] = hi.w * inv;
        }
        float cs[8], sn[8];
#pragma unroll
        for (int c = 0; c < 8; c += 2) {
            const float4 t4 = *(const float4*)&a.rope[((size_t)m * 32 + j0 + c) * 2];
            cs[c] = t4.x; sn[c] = t4.y; cs[c + 1] = t4.z; sn[c + 1] = t4.w;
        }
        float* kT = a.kc + (size_t)(n0 >> 6) * 64 * a.MS;
        float* qr = a.p[0].C + (size_t)m * ldc + n0;
#pragma unroll
        for (int c = 0; c < 8; c += 4) {
            float e0[4], e1[4];
#pragma unroll
            for (int q = 0; q < 4; q++) {
                e0[q] = k0[c + q] * cs[c + q] - k1[c + q] * sn[c + q];
                e1[q] = k0[c + q] * sn[c + q] + k1[c + q] * cs[c + q];
            }
            if (p == 0) {
                *(float4*)&qr[j0 + c] = make_float4(e0[0], e0[1], e0[2], e0[3]);
                *(float4*)&qr[32 + j0 + c] = make_float4(e1[0], e1[1], e1[2], e1[3]);
            } else {
                *(float4*)&kT[((size_t)((j0 + c) >> 2) * a.MS + m) * 4] = make_float4(e0[0], e0[1], e0[2], e0[3]);
                *(float4*)&kT[((size_t)((32 + j0 + c) >> 2) * a.MS + m) * 4] =
                    make_float4(e1[0], e1[1], e1[2], e1[3]);
            }
        }
    } else {
        float xn[CPT]; /* the stored values (x after the residual add); 0 past N */
#pragma unroll
        for (int c = 0; c < CPT; c += 4) {
            float4 v = *(const float4*)&part[0][r][c0 + c];
#pragma unroll
            for (int w = 1; w < 4; w++) {
                const float4 pw = *(const float4*)&part[w][r][c0 + c];
                v.x += pw.x; v.y += pw.y; v.z += pw.z; v.w += pw.w;
            }
            if (EPI != PFG_RESID) {
                v.x *= inv; v.y *= inv; v.z *= inv; v.w *= inv;
            }
            float vv[4] = {v.x, v.y, v.z, v.w};
            if (whole) {
                if (EPI == PFG_RESID) {
                    const float4 o = res[c >> 2];
                    vv[0] += o.x; vv[1] += o.y; vv[2] += o.z; vv[3] += o.w;
                }
                const f32x4 v4 = {vv[0], vv[1], vv[2], vv[3]};
                __builtin_nontemporal_store(v4, (f32x4*)&dst[c]);
            } else {
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    if (n0 + c0 + c + e < N) {
                        if (EPI == PFG_RESID) vv[e] += dst[c + e];
                        dst[c + e] = vv[e];
                    } else {
                        vv[e] = 0.f;
                    }
                }
            }
#pragma unroll
            for (int e = 0; e < 4; e++) xn[c + e] = vv[e];
        }
        if (EPI == PFG_RESID && a.an) {
            /* the next RMSNorm's operand and this tile's partial sum of squares */
            float ss = 0.f;
#pragma unroll
            for (int c = 0; c < CPT; c++) ss = fmaf(xn[c], xn[c], ss);
            ss += __shfl_xor(ss, 1);
            ss += __shfl_xor(ss, 2); /* the four threads of row r */
            if ((t & 3) == 0) a.ss_out[(size_t)nt * a.ss_ld + m] = ss;
            const int nks = (N + 63) >> 6;
#pragma unroll
            for (int hf = 0; hf < CPT / 8; hf++) {
                unsigned int w[4];
#pragma unroll
                for (int c = 0; c < 8; c += 2) {
                    const int cc = n0 + c0 + 8 * hf + c;
                    const float lo = cc < N ? xn[8 * hf + c] * gnr[8 * hf + c] : 0.f;
                    const float hi = cc + 1 < N ? xn[8 * hf + c + 1] * gnr[8 * hf + c + 1] : 0.f;
                    w[c >> 1] = pk2(lo, hi);
                }
                *(uint4*)(a.an + frag_index(m, n0 + c0 + 8 * hf, nks)) = make_uint4(w[0], w[1], w[2], w[3]);
            }
        }
    }
}

/* One lane slot of one chunk of the prefill weight layout per thread. */
template <int QF>
__global__ __launch_bounds__(PNTH) void k_pfg_repack(const unsigned char* __restrict__ src, unsigned char* __restrict__ dst,
                                                    int N, int nkb, int ns, long nslots) {
    constexpr unsigned BYTES = QFmt<QF>::BYTES;
    constexpr unsigned CH = QF == QF_Q4 ? PFG_CHUNK_Q4 : PFG_CHUNK_Q8;
    const long i = (long)blockIdx.x * PNTH + threadIdx.x;
    if (i >= nslots) return;
    const int lane = (int)(i & 63);
    const long ch = i >> 6;
    const int s = (int)(ch % ns);
    const long row = 32 * (ch / ns) + (lane & 31);
    const int blk = 2 * s + (lane >> 5);
    float sc = 0.f;
    uint4 q0 = make_uint4(0u, 0u, 0u, 0u), q1 = q0;
    if (row < N && blk < nkb) {
        const unsigned char* b = src + ((size_t)row * nkb + blk) * BYTES;
        __builtin_memcpy(&sc, __builtin_assume_aligned(b, 4), 4);
        __builtin_memcpy(&q0, __builtin_assume_aligned(b + 4, 4), 16);
        if (QF == QF_Q8) __builtin_memcpy(&q1, __builtin_assume_aligned(b + 20, 4), 16);
    }
    unsigned char* c = dst + (size_t)ch * CH;
    *(float*)(c + 4 * lane) = sc;
    *(uint4*)(c + 256 + 16 * lane) = q0;
    if (QF == QF_Q8) *(uint4*)(c + 1280 + 16 * lane) = q1;
}

} // namespace

extern "C" size_t pfg_wbytes(int N, int K, int qf) {
    return (size_t)((N + 31) / 32) * ((K + 63) / 64) * (qf ? PFG_CHUNK_Q4 : PFG_CHUNK_Q8);
}

extern "C" int pfg_repack(const unsigned char* src, unsigned char* dst, int N, int K, int qf, hipStream_t s) {
    BMK_REQUIRE(N > 0 && K > 0 && K % 32 == 0, "pfg_repack: N %d, K %d", N, K);
    BMK_REQUIRE(((uintptr_t)src & 3) == 0 && ((uintptr_t)dst & 15) == 0, "pfg_repack: misaligned operands");
    const int ns = (K + 63) / 64;
    const long nslots = (long)((N + 31) / 32) * ns * 64;
    const dim3 grid((unsigned)((nslots + PNTH - 1) / PNTH));
    if (qf) hipLaunchKernelGGL(k_pfg_repack<QF_Q4>, grid, dim3(PNTH), 0, s, src, dst, N, K / 32, ns, nslots);
    else hipLaunchKernelGGL(k_pfg_repack<QF_Q8>, grid, dim3(PNTH), 0, s, src, dst, N, K / 32, ns, nslots);
    BMK_LAUNCH_CHECK();
    return 0;
}

extern "C" int pfg_launch(PfgArgs* a, int qf, int epi, hipStream_t s) {
    BMK_REQUIRE(a->M > 0 && a->K > 0 && a->K % 32 == 0, "pf_gemm: M %d, K %d (K a multiple of 32)", a->M, a->K);
    BMK_REQUIRE(a->nprob >= 1 && a->nprob <= PFG_MAX_PROBS, "pf_gemm: %d problems", a->nprob);
    BMK_REQUIRE(epi == PFG_STORE || (epi == PFG_RESID && a->nprob == 1 && a->x) ||
                    (epi == PFG_SWIGLU && a->nprob == 2 && a->h && a->p[0].N == a->p[1].N) ||
                    (epi == PFG_QKV && a->nprob == 3 && a->kc && a->vc && a->rope && a->M <= a->MS &&
                     a->p[1].N == a->p[2].N && ((uintptr_t)a->rope & 15) == 0 &&
                     a->p[0].N % 64 == 0 && a->p[1].N % 64 == 0 && a->p[0].ldc % 4 == 0 &&
                     ((uintptr_t)a->p[0].C & 15) == 0 && ((uintptr_t)a->kc & 15) == 0 && ((uintptr_t)a->vc & 15) == 0),
                "pf_gemm: epilogue %d does not fit its %d problems", epi, a->nprob);
    BMK_REQUIRE(((uintptr_t)a->A & 15) == 0 && ((uintptr_t)a->W & 15) == 0 && ((uintptr_t)a->h & 15) == 0 &&
                    ((uintptr_t)a->an & 15) == 0,
                "pf_gemm: activations, weights and bf16 outputs must be 16-byte aligned");
    BMK_REQUIRE(!a->ss_in || (epi != PFG_RESID && a->ss_tiles > 0 && a->ss_tiles <= PFG_SS_MAX && a->ss_ld >= a->M &&
                              a->norm_d > 0),
                "pf_gemm: RMSNorm scale of the rows needs its partial sums");
    BMK_REQUIRE(!a->an || (epi == PFG_RESID && a->gn && a->ss_out && a->ss_ld >= a->M),
                "pf_gemm: the next RMSNorm's operand comes from a residual launch with its weights and sums");
    /* Tiles: 32 rows (one row fragment per wave) halve each workgroup's
     * chain (512 tokens: 6.4-6.7 against 7.8-8.1 us per launch), unless the
     * launch would then need more than two workgroups per CU.  A residual
     * launch of fewer than 128 such tiles also narrows them to 32 columns
     * (its epilogue has no column pairs; its row sums then come in N / 32
     * parts): 128 tokens 5.9 -> 4.5 us; at 512 tokens no change. */
    /* (32-column tiles of a residual launch cover whole 64-column steps, so
     * that the next norm's operand gets its zero padding from the last) */
    auto tiles_of = [&](int N, int tw) { return tw == 32 ? 2 * ((N + 63) / 64) : (N + tw - 1) / tw; };
    auto count_tiles = [&](int tw) {
        int n = 0;
        for (int i = 0; i < a->nprob; i++) n += tiles_of(a->p[i].N, tw);
        return epi == PFG_SWIGLU ? 2 * ((a->p[0].N + 63) / 64) : n;
    };
    const long mt32 = (a->M + 31) / 32;
    const int nj = epi == PFG_RESID && mt32 * count_tiles(64) < 128 && count_tiles(32) <= PFG_SS_MAX ? 1 : 2;
    const int tw = 32 * nj;
    const int mi = mt32 * count_tiles(tw) > 512 ? 2 : 1;
    int nt = 0;
    for (int i = 0; i < a->nprob; i++) {
        BMK_REQUIRE(a->p[i].N > 0, "pf_gemm: problem %d has N = %d", i, a->p[i].N);
        BMK_REQUIRE(epi == PFG_SWIGLU || a->p[i].ldc >= a->p[i].N, "pf_gemm: ldc %d < N %d", a->p[i].ldc, a->p[i].N);
        BMK_REQUIRE((epi != PFG_STORE && !(epi == PFG_QKV && i == 0)) || a->p[i].C, "pf_gemm: problem %d has no output",
                    i);
        BMK_REQUIRE((a->p[i].w_off & 15) == 0, "pf_gemm: weight offset not 16-byte aligned");
        a->p[i].tile0 = nt;
        if (epi != PFG_SWIGLU) nt += tiles_of(a->p[i].N, tw);
    }
    if (epi == PFG_SWIGLU) nt = 2 * ((a->p[0].N + 63) / 64); /* every 64-column step of h, padding included */
    a->NT = nt;
    const long grid = (long)((a->M + 32 * mi - 1) / (32 * mi)) * nt;
    BMK_REQUIRE(grid > 0 && grid < (1L << 31), "pf_gemm: %ld workgroups", grid);
#define PFG_GO(Q, E)                                                                                          \
    do {                                                                                                      \
        if (mi == 1) hipLaunchKernelGGL((k_pf_gemm<Q, E, 1, 2>), dim3((unsigned)grid), dim3(PNTH), 0, s, *a);  \
        else hipLaunchKernelGGL((k_pf_gemm<Q, E, 2, 2>), dim3((unsigned)grid), dim3(PNTH), 0, s, *a);          \
    } while (0)
#define PFG_GO_R(Q)                                                                                           \
    do {                                                                                                      \
        if (nj == 2) PFG_GO(Q, PFG_RESID);                                                                    \
        else if (mi == 1) hipLaunchKernelGGL((k_pf_gemm<Q, PFG_RESID, 1, 1>), dim3((unsigned)grid), dim3(PNTH), 0, s, *a); \
        else hipLaunchKernelGGL((k_pf_gemm<Q, PFG_RESID, 2, 1>), dim3((unsigned)grid), dim3(PNTH), 0, s, *a);  \
    } while (0)
    if (qf) {
        if (epi == PFG_STORE) PFG_GO(QF_Q4, PFG_STORE);
        else if (epi == PFG_RESID) PFG_GO_R(QF_Q4);
        else if (epi == PFG_QKV) PFG_GO(QF_Q4, PFG_QKV);
        else PFG_GO(QF_Q4, PFG_SWIGLU);
    } else {
        if (epi == PFG_STORE) PFG_GO(QF_Q8, PFG_STORE);
        else if (epi == PFG_RESID) PFG_GO_R(QF_Q8);
        else if (epi == PFG_QKV) PFG_GO(QF_Q8, PFG_QKV);
        else PFG_GO(QF_Q8, PFG_SWIGLU);
    }
#undef PFG_GO
#undef PFG_GO_R
    BMK_LAUNCH_CHECK();
    return 0;
}
