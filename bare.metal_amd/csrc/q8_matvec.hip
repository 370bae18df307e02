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
#include <vector>

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
 * A workgroup is BMV_WAVES waves; it runs the plan tile tile_map[blockIdx.x]
 * (problem << 16 | tile, from bm_q8_bmv_plan: each XCD's workgroups take
 * whole problems, longest rows first) for batch rows 16*blockIdx.y .. +15
 * (8 when BT <= 8) over the whole K range.  A tile is BMV_TILE_ROWS rows:
 * BMV_SUBTILES sub-tiles of 16 rows per wave.  K runs in chunks of CB
 * blocks; per chunk the workgroup splits the chunk's activations once into
 * LDS and every sub-tile's steps use them.  Weights never pass through LDS:
 *   - per step of 8 K blocks, lane (c = l%16, h = l/16) of a wave loads
 *     whole blocks h and 4 + h of its row c (a dwordx4, a dwordx4 and a
 *     dword each), so a wave streams 288 contiguous bytes of each of its
 *     16 rows per step: few rows at a time, long runs in each, which is
 *     what keeps HBM near its streaming rate (64 rows per wave with
 *     144-byte runs streamed at 42% of the peak, 16 rows with 288-byte
 *     runs at 73-76%, loads alone); loads run BMV_WSTAGES steps ahead in
 *     registers of their own;
 *   - a 4x4 transpose over the lane quarters (v_permlane32_swap, then
 *     v_permlane16_swap) leaves lane (c, g) holding codes 8g .. 8g+7 of
 *     row c for each of a quad's 4 blocks: the MFMA B operand, with no LDS
 *     store, barrier or bank conflict; the block scales are gathered
 *     across the quarters the same way;
 *   - each activation is split exactly into three bf16 terms (split3) and
 *     stored in LDS in the MFMA A-operand order, so the split is paid once
 *     per BMV_TILE_ROWS output rows; a barrier before a chunk's products
 *     and one after them are the only workgroup barriers.
 * Every product is exact, so each block sum is an fp32 sum of the exact
 * x * q products, as in the fp32 reference (only the order differs).  Each
 * block product is scaled by its row's block scale and added in block
 * order, as the reference scales each block's dot product
 * (forward.metal:575-623).  D layout: lane l holds batch rows 4*(l/16)+v of
 * output row l%16.  Problem p reads BT rows of C floats at X + x_off (row
 * stride C) and writes BT rows of OC floats at Y + y_off (row stride OC). */
typedef float bmm_f32x4 __attribute__((ext_vector_type(4)));
typedef float bmm_f32x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bmm_bf16x8 __attribute__((ext_vector_type(8)));
constexpr int BMV_QUADS = 2; /* quads of 4 K blocks per step */

/* x = hi + mid + lo with three bf16 terms: hi keeps the top 8 significant
 * bits of x (truncated, so no term overflows), mid the top 8 of x - hi and
 * lo the at most 8 bits left; both subtractions are exact in fp32, so the
 * split is exact for every finite x whose lowest significant bit lies at or
 * above bf16's smallest normal (|x| >= 2^-102 suffices).  Each term pair is
 * packed by one v_perm_b32 (the upper halves of two fp32 words).  Returns
 * the lanes of the wave with a value that is not finite: those need
 * split3_exact. */
__device__ __forceinline__ unsigned int hi16_pair(unsigned int lo_word, unsigned int hi_word) {
    return __builtin_amdgcn_perm(hi_word, lo_word, 0x07060302u);
}
__device__ __forceinline__ unsigned long long split3(const bmm_f32x8& x, uint4& hi, uint4& mid, uint4& lo) {
    unsigned int u[8], m[8], l[8];
    unsigned long long nf = 0; /* lanes of the wave holding a non-finite value (one v_cmp_class each) */
#pragma unroll
    for (int i = 0; i < 8; i++) {
        u[i] = __float_as_uint(x[i]);
        nf |= __builtin_amdgcn_ballot_w64(!__builtin_isfinite(x[i]));
        const float r1 = x[i] - __uint_as_float(u[i] & 0xffff0000u);
        m[i] = __float_as_uint(r1);
        l[i] = __float_as_uint(r1 - __uint_as_float(m[i] & 0xffff0000u));
    }
    hi = make_uint4(hi16_pair(u[0], u[1]), hi16_pair(u[2], u[3]), hi16_pair(u[4], u[5]), hi16_pair(u[6], u[7]));
    mid = make_uint4(hi16_pair(m[0], m[1]), hi16_pair(m[2], m[3]), hi16_pair(m[4], m[5]), hi16_pair(m[6], m[7]));
    lo = make_uint4(hi16_pair(l[0], l[1]), hi16_pair(l[2], l[3]), hi16_pair(l[4], l[5]), hi16_pair(l[6], l[7]));
    return nf;
}
/* The same split with non-finite values handled: a non-finite x goes
 * whole into hi (a NaN kept a NaN) with mid = lo = 0, so its products are
 * the fp32 ones (Inf * 0 = NaN, Inf * q = Inf). */
__device__ __forceinline__ void split3_exact(const bmm_f32x8& x, uint4& hi, uint4& mid, uint4& lo) {
    unsigned int u[8], m[8], l[8];
#pragma unroll
    for (int i = 0; i < 8; i++) {
        u[i] = __float_as_uint(x[i]);
        const bool fin = __builtin_isfinite(x[i]);
        const float r1 = fin ? x[i] - __uint_as_float(u[i] & 0xffff0000u) : 0.0f;
        if (!fin && (u[i] & 0x007fffffu)) u[i] |= 0x00400000u;
        m[i] = __float_as_uint(r1);
        l[i] = __float_as_uint(r1 - __uint_as_float(m[i] & 0xffff0000u));
    }
    hi = make_uint4(hi16_pair(u[0], u[1]), hi16_pair(u[2], u[3]), hi16_pair(u[4], u[5]), hi16_pair(u[6], u[7]));
    mid = make_uint4(hi16_pair(m[0], m[1]), hi16_pair(m[2], m[3]), hi16_pair(m[4], m[5]), hi16_pair(m[6], m[7]));
    lo = make_uint4(hi16_pair(l[0], l[1]), hi16_pair(l[2], l[3]), hi16_pair(l[4], l[5]), hi16_pair(l[6], l[7]));
}

/* Exchange between lane halves / quarters (gfx950 v_permlane32_swap:
 * lanes 32..63 of a with lanes 0..31 of b; v_permlane16_swap: lanes 16..31
 * of a with lanes 0..15 of b, and lanes 48..63 of a with 32..47 of b). */
__device__ __forceinline__ void swap32(unsigned int& a, unsigned int& b) {
    const auto r = __builtin_amdgcn_permlane32_swap(a, b, false, false);
    a = r[0];
    b = r[1];
}
__device__ __forceinline__ void swap16(unsigned int& a, unsigned int& b) {
    const auto r = __builtin_amdgcn_permlane16_swap(a, b, false, false);
    a = r[0];
    b = r[1];
}

/* One quad of one 16-row group in registers: lane (c, h) holds the scale
 * and code dwords of block h of row c; after bmv_transpose, code dwords
 * CW*u .. CW*u+CW-1 are codes 8g .. 8g+7 of block u for lane (c, g) and
 * s[u] is block u's scale of row c. */
template <int QF> struct BmvQuad {
    static constexpr int CW = QF == QF_Q8 ? 2 : 1; /* dwords per 8 codes */
    unsigned int s[4];
    unsigned int d[4 * CW];
};

template <int QF>
__device__ __forceinline__ void bmv_load(BmvQuad<QF>& Q, const unsigned char* p) {
    if (QF == QF_Q8) {
        uint4 a, b;
        __builtin_memcpy(&a, __builtin_assume_aligned(p, 4), 16);
        __builtin_memcpy(&b, __builtin_assume_aligned(p + 16, 4), 16);
        __builtin_memcpy(&Q.d[7], __builtin_assume_aligned(p + 32, 4), 4);
        Q.s[0] = a.x;
        Q.d[0] = a.y; Q.d[1] = a.z; Q.d[2] = a.w;
        Q.d[3] = b.x; Q.d[4] = b.y; Q.d[5] = b.z; Q.d[6] = b.w;
    } else {
        uint4 a;
        __builtin_memcpy(&Q.s[0], __builtin_assume_aligned(p, 4), 4);
        __builtin_memcpy(&a, __builtin_assume_aligned(p + 4, 4), 16);
        Q.d[0] = a.x; Q.d[1] = a.y; Q.d[2] = a.z; Q.d[3] = a.w;
    }
}

/* The 4x4 transpose of 8-code pieces (row = lane quarter, column = piece)
 * and the all-gather of the quarter's scales, both in two swap stages. */
template <int QF>
__device__ __forceinline__ void bmv_transpose(BmvQuad<QF>& Q) {
    constexpr int CW = BmvQuad<QF>::CW;
#pragma unroll
    for (int e = 0; e < 2 * CW; e++) swap32(Q.d[e], Q.d[2 * CW + e]);
#pragma unroll
    for (int e = 0; e < CW; e++) {
        swap16(Q.d[e], Q.d[CW + e]);
        swap16(Q.d[2 * CW + e], Q.d[3 * CW + e]);
    }
    unsigned int b = Q.s[0];
    swap32(Q.s[0], b); /* quarters 0..3: s[0] = s0 s1 s0 s1, b = s2 s3 s2 s3 */
    Q.s[1] = Q.s[0];
    Q.s[3] = b;
    swap16(Q.s[0], Q.s[1]);
    Q.s[2] = b;
    swap16(Q.s[2], Q.s[3]);
}

/* codes 8g .. 8g+7 of block u as the bf16 B operand (exact) */
template <int QF>
__device__ __forceinline__ bmm_bf16x8 bmv_codes(const BmvQuad<QF>& Q, int u) {
    bmm_f32x8 w;
    if (QF == QF_Q4) {
        const unsigned int q0 = Q.d[u];
#pragma unroll
        for (int i = 0; i < 8; i++) w[i] = q4_code(q0, i);
    } else {
        const unsigned int q0 = Q.d[2 * u], q1 = Q.d[2 * u + 1];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            w[i] = q8_byte(q0, i);
            w[4 + i] = q8_byte(q1, i);
        }
    }
    return __builtin_convertvector(w, bmm_bf16x8);
}

/* A-operand layouts of the batched kernel, per K block:
 *   NSLOT 1 (at most 8 batch rows): A1 = [hi of rows 0..7; mid of rows
 *     0..7], A2 = [lo of rows 0..7; zeros]: two MFMAs per block, rows 8..15
 *     of D carry the mid products of rows 0..7, added at the end;
 *   NSLOT 2 (up to 16 rows): hi, mid and lo of all 16 rows: three MFMAs.
 * Slot s of a block's area is 16 bytes: 8 bf16 of one A row. */
template <int NSLOT> struct BmvA;
template <> struct BmvA<1> {
    static constexpr int TERMS = 2, SLOTS = 64 + 33; /* A1: slot r + 16g; A2: slot r + 8g (r < 8), 32 = zeros */
    static constexpr int CB = BMV_CB;                 /* K blocks per activation chunk */
};
template <> struct BmvA<2> {
    static constexpr int TERMS = 3, SLOTS = 3 * 64;   /* term t: slot 64t + r + 16g */
    static constexpr int CB = BMV_CB;
};

template <int QF, int NSLOT>
__global__ __launch_bounds__(64 * BMV_WAVES) void k_bmv_multi(const unsigned char* __restrict__ W,
                                                              const float* __restrict__ X, float* __restrict__ Y,
                                                              const MvDesc* __restrict__ desc,
                                                              const unsigned int* __restrict__ tile_map, int n_tiles,
                                                              int BT) {
    typedef BmvA<NSLOT> L;
    constexpr int BYTES = QFmt<QF>::BYTES;
    constexpr int KS = 4 * BMV_QUADS;    /* K blocks per step */
    constexpr int AR = 8 * NSLOT;        /* batch rows per launch tile */
    constexpr int CB = L::CB;            /* K blocks per activation chunk */
    constexpr int SPC = CB / KS;         /* steps per sub-tile and chunk */
    constexpr int T = BMV_SUBTILES;      /* 16 x BMV_WAVES-row sub-tiles of a plan tile */
    constexpr int XSL = CB * 4 * AR / (64 * BMV_WAVES); /* 8-column activation slots per lane and chunk */
    static_assert(XSL * 64 * BMV_WAVES == CB * 4 * AR, "chunk shape");
    __shared__ uint4 xs[CB][L::SLOTS];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int c = lane & 15, h = lane >> 4;
    const int b0 = AR * (int)blockIdx.y;
    const int nbt = min(AR, BT - b0); /* batch rows of this launch tile */
    if (NSLOT == 1 && tid < CB) xs[tid][64 + 32] = make_uint4(0u, 0u, 0u, 0u);

    /* A workgroup runs the plan tile tile_map[blockIdx.x] = (problem << 16)
     * | tile (or nothing: BMV_IDLE_TILE), chunk after chunk; within a chunk,
     * sub-tile after sub-tile (wave w: rows 16w .. 16w+15 of each), all on
     * the chunk's one staging of the activations.  Cur is one chunk; past
     * the last, it reads its loads at the tile's first bytes and computes
     * nothing. */
    const unsigned int m = tile_map[blockIdx.x];
    if (m == BMV_IDLE_TILE) return;
    const MvDesc d = desc[m >> 16];
    struct Cur {
        int ch;
        bool live;
    };
    const int nb = d.C / 32;
    const int nch = (nb + CB - 1) / CB;
    const int row0 = (int)(m & 0xffffu) * BMV_TILE_ROWS + 16 * wave; /* in sub-tile 0 */
    auto advance = [&](Cur& k) {
        k.ch++;
        k.live = k.ch < nch;
    };

    /* Weight loads of step s2 of sub-tile j of chunk k, lane (c, h): whole
     * blocks h and 4 + h of the step's 8 of its row c.  Every lane issues
     * the same loads whatever the step; a block past the row (or a row or
     * chunk past the end) reads the tile's first block instead (one line
     * for the whole wave; its product is skipped), so no branch separates
     * two steps' loads. */
    auto load_w = [&](BmvQuad<QF> (&S)[BMV_QUADS], const Cur& k, int j, int s2) {
        const unsigned char* wp = W + d.w_off;
        const int row = row0 + 16 * BMV_WAVES * j + c;
        const unsigned int roff = (unsigned int)row * (unsigned int)(nb * BYTES);
        const bool on = k.live && row < d.OC;
#pragma unroll
        for (int u = 0; u < BMV_QUADS; u++) {
            const int kb = CB * k.ch + KS * s2 + 4 * u + h;
            bmv_load<QF>(S[u], wp + (on && kb < nb ? roff + (unsigned int)kb * BYTES : 0u));
        }
    };

    /* Activations of chunk k: slot i = tid + 256 r of the chunk's AR x 4*CB
     * slots is batch row i % AR (a row past the batch reads row 0: it only
     * reaches output rows that are never stored), 8-column group i / AR (a
     * group past the row reads the row's first columns: its blocks are
     * skipped).  load_x issues them a chunk ahead, into registers of their
     * own, so that waiting for them never waits for the weight loads issued
     * after them. */
    struct XChunk {
        float4 a[XSL], b[XSL];
    };
    auto load_x = [&](XChunk& Xc, const Cur& k) {
#pragma unroll
        for (int r = 0; r < XSL; r++) {
            const int i = tid + 64 * BMV_WAVES * r, b = i % AR, g8 = i / AR;
            const int col = 32 * CB * k.ch + 8 * g8;
            const size_t o = k.live ? (size_t)(b0 + (b < nbt ? b : 0)) * (size_t)d.C + (col < d.C ? col : 0) : 0;
            const float* p = X + d.x_off + o;
            __builtin_memcpy(&Xc.a[r], __builtin_assume_aligned(p, 16), 16);
            __builtin_memcpy(&Xc.b[r], __builtin_assume_aligned(p + 4, 16), 16);
        }
    };
    /* Split into LDS.  The exact split of non-finite values runs, and
     * rewrites the slots, only when some lane of the wave holds one: a
     * branch around stores, which the compiler keeps as a branch. */
    auto put = [&](int u, int b, int g, const uint4& th, const uint4& tm, const uint4& tl) {
        if (NSLOT == 1) {
            xs[u][b + 16 * g] = th;
            xs[u][b + 8 + 16 * g] = tm;
            xs[u][64 + b + 8 * g] = tl;
        } else {
            xs[u][b + 16 * g] = th;
            xs[u][64 + b + 16 * g] = tm;
            xs[u][128 + b + 16 * g] = tl;
        }
    };
    auto stage_x = [&](const XChunk& Xc) {
#pragma unroll
        for (int r = 0; r < XSL; r++) {
            const int i = tid + 64 * BMV_WAVES * r, b = i % AR, g8 = i / AR, u = g8 >> 2, g = g8 & 3;
            uint4 th, tm, tl;
            const bmm_f32x8 xf = {Xc.a[r].x, Xc.a[r].y, Xc.a[r].z, Xc.a[r].w, Xc.b[r].x, Xc.b[r].y, Xc.b[r].z, Xc.b[r].w};
            const unsigned long long nf = split3(xf, th, tm, tl);
            put(u, b, g, th, tm, tl);
            if (nf) {
                split3_exact(xf, th, tm, tl);
                put(u, b, g, th, tm, tl);
            }
        }
    };

    bmm_f32x4 acc[T];
#pragma unroll
    for (int j = 0; j < T; j++) acc[j] = bmm_f32x4{0.f, 0.f, 0.f, 0.f};
    /* this lane's A slots: NSLOT 1: A1 row c (hi of row c, or mid of row
     * c - 8), A2 row c (lo of row c, or zeros); NSLOT 2: row c of each term */
    const int a_slot0 = c + 16 * h;
    const int a_slot1 = NSLOT == 1 ? (c < 8 ? 64 + c + 8 * h : 64 + 32) : 64 + c + 16 * h;
    const int a_slot2 = 128 + c + 16 * h;

    /* The products of step s2 of chunk k from registers S and the chunk's
     * LDS operands into A, block after block (the waves of a SIMD hide each
     * other's MFMA latency; one block's operands at a time keeps the
     * registers for loads in flight). */
    auto compute = [&](BmvQuad<QF> (&S)[BMV_QUADS], const Cur& k, int s2, bmm_f32x4& A) {
        const int kb0 = CB * k.ch + KS * s2; /* the step's first block */
        const int nb_ = nb;
#pragma unroll
        for (int u = 0; u < BMV_QUADS; u++) bmv_transpose<QF>(S[u]);
#pragma unroll
        for (int p = 0; p < KS; p++) {
            /* blocks past the row (the same for the whole wave) are skipped,
             * not weighted by 0: 0 * Inf would be NaN */
            if (kb0 + p >= nb_) break;
            bmm_bf16x8 xa[L::TERMS];
#pragma unroll
            for (int t = 0; t < L::TERMS; t++) {
                const uint4 a = xs[KS * s2 + p][t == 0 ? a_slot0 : t == 1 ? a_slot1 : a_slot2];
                __builtin_memcpy(&xa[t], &a, 16);
            }
            const bmm_bf16x8 wv = bmv_codes<QF>(S[p >> 2], p & 3);
            bmm_f32x4 dd = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xa[0], wv, bmm_f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
#pragma unroll
            for (int t = 1; t < L::TERMS; t++) dd = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xa[t], wv, dd, 0, 0, 0);
            const float sc = __uint_as_float(S[p >> 2].s[p & 3]);
#pragma unroll
            for (int v = 0; v < 4; v++) A[v] = fmaf(sc, dd[v], A[v]);
        }
    };

    /* Every wave issues its weight loads, a wave past the last row too (its
     * lanes read the tile's first block): a load behind a branch makes the
     * compiler wait for every earlier load at the join.  Weights stream
     * BMV_WSTAGES steps ahead in (chunk, sub-tile, step) order, across
     * sub-tile, chunk and tile boundaries; per chunk, the workgroup
     * stages the chunk's activations (loaded during the previous chunk)
     * before a barrier, and a barrier after the chunk's products frees the
     * LDS for the next.  Scheduling barriers keep every load group where it
     * stands in program order: the compiler would otherwise sink a stage's
     * loads below the next step's products, and the next step would then
     * wait for both sets.  Nothing between two waits may itself wait for a
     * load (a spilled register reloaded, say): loads complete in order, so
     * that wait would drain every weight load in flight. */
    /* NS register sets: the steps of a chunk (T sub-tiles x SPC steps) take
     * them in turn, the loads of step f going to step f + NS */
    constexpr int NS = BMV_WSTAGES;
    constexpr int FPC = T * SPC; /* steps per chunk */
    static_assert(FPC % NS == 0, "register sets cycle within a chunk");
    BmvQuad<QF> w[NS][BMV_QUADS];
    XChunk xn;
    Cur cur = {0, true}, nxt = cur;
    advance(nxt);
    load_x(xn, cur);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int f = 0; f < NS; f++) load_w(w[f], cur, f / SPC, f % SPC);
    __builtin_amdgcn_sched_barrier(0);
    while (cur.live) {
        stage_x(xn);
        __builtin_amdgcn_sched_barrier(0);
        load_x(xn, nxt);
        __builtin_amdgcn_sched_barrier(0);
        __syncthreads();
#pragma unroll
        for (int f = 0; f < FPC; f++) {
            const int j = f / SPC, s2 = f % SPC;
            /* the same for the whole wave */
            const bool sub_live = row0 + 16 * BMV_WAVES * j < d.OC;
            if (sub_live && CB * cur.ch + KS * s2 < nb) compute(w[f % NS], cur, s2, acc[j]);
            __builtin_amdgcn_sched_barrier(0);
            /* the step NS ahead: in this chunk, or in the next */
            const int f2 = f + NS;
            if (f2 < FPC) load_w(w[f % NS], cur, f2 / SPC, f2 % SPC);
            else load_w(w[f % NS], nxt, (f2 - FPC) / SPC, (f2 - FPC) % SPC);
            __builtin_amdgcn_sched_barrier(0);
        }
        cur = nxt;
        advance(nxt);
        __syncthreads();
    }
#pragma unroll
    for (int j = 0; j < T; j++) {
        const int row = row0 + 16 * BMV_WAVES * j + c;
        bmm_f32x4 yv = acc[j];
        if (NSLOT == 1) {
            /* D rows 8..15 (lanes 32..63) carry the mid products of rows 0..7 */
#pragma unroll
            for (int v = 0; v < 4; v++) {
                unsigned int lo_half = __float_as_uint(yv[v]), hi_half = lo_half;
                swap32(lo_half, hi_half); /* lanes 0..31 now see lanes 32..63's value in hi_half */
                yv[v] += __uint_as_float(hi_half);
            }
        }
        if (row < d.OC && (NSLOT == 2 || h < 2)) {
            float* y = Y + d.y_off + row;
#pragma unroll
            for (int v = 0; v < 4; v++) {
                const int b = b0 + 4 * h + v;
                if (b < BT) y[(size_t)b * d.OC] = yv[v];
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
    /* at most 8 rows: one launch tile of 8 rows; above: tiles of 16 rows */
    const dim3 grid((unsigned)n_tiles, (unsigned)(BT <= 8 ? 1 : (BT + 15) / 16)), tb(64 * BMV_WAVES);
    if (qf == QF_Q4) {
        if (BT <= 8) hipLaunchKernelGGL((k_bmv_multi<QF_Q4, 1>), grid, tb, 0, s, W, X, Y, d_desc, d_tile_map, n_tiles, BT);
        else hipLaunchKernelGGL((k_bmv_multi<QF_Q4, 2>), grid, tb, 0, s, W, X, Y, d_desc, d_tile_map, n_tiles, BT);
    } else {
        if (BT <= 8) hipLaunchKernelGGL((k_bmv_multi<QF_Q8, 1>), grid, tb, 0, s, W, X, Y, d_desc, d_tile_map, n_tiles, BT);
        else hipLaunchKernelGGL((k_bmv_multi<QF_Q8, 2>), grid, tb, 0, s, W, X, Y, d_desc, d_tile_map, n_tiles, BT);
    }
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
    /* BT == 1: every problem owns the run of workgroups tile_map[t] == i for
     * t in [tile0, tile0 + tiles), the runs in problem order.  BT >= 2: each
     * tile-map entry names (problem << 16) | tile or is BMV_IDLE_TILE, and
     * every tile of every problem appears exactly once. */
    long next_tile = 0;
    for (int i = 0; i < nprob; i++) {
        const MvDesc& d = desc[i];
        BMK_REQUIRE(d.OC > 0 && d.C > 0 && d.C % 32 == 0, "q8 matvec multi: problem %d bad shape OC=%d C=%d", i, d.OC, d.C);
        const int want = BT > 1 ? bm_q8_bmv_tiles(d.OC, d.C) : mv_tiles_for(d.OC, d.C, U);
        BMK_REQUIRE(d.tiles == want && (BT > 1 || d.tile0 == next_tile),
                    "q8 matvec multi: problem %d tiles %d@%d, expected %d@%ld", i, d.tiles, d.tile0, want, next_tile);
        BMK_REQUIRE((d.w_off & 3) == 0, "q8 matvec multi: problem %d weight offset not 4-byte aligned", i);
        /* the batched kernel addresses a problem's rows with 32-bit offsets */
        BMK_REQUIRE(BT == 1 || (unsigned long long)d.OC * (d.C / 32) * BYTES <= 0xffffffffull,
                    "q8 matvec multi: problem %d spans 4 GiB or more", i);
        /* the batched kernel loads activations 16 bytes at a time */
        BMK_REQUIRE(BT == 1 || (d.x_off & 3) == 0, "q8 matvec multi: problem %d activation offset not 16-byte aligned", i);
        BMK_REQUIRE(d.w_off + (unsigned long long)d.OC * (d.C / 32) * BYTES <= a->bytes[2] &&
                    d.x_off + (unsigned long long)BT * d.C <= a->bytes[3] / 4 &&
                    d.y_off + (unsigned long long)BT * d.OC <= a->bytes[4] / 4,
                    "q8 matvec multi: problem %d lies outside its arenas", i);
        next_tile += d.tiles;
    }
    if (BT == 1) {
        BMK_REQUIRE(next_tile == n_tiles, "q8 matvec multi: tiles sum to %ld, n_tiles=%d", next_tile, n_tiles);
        for (int i = 0; i < nprob; i++)
            for (int t = desc[i].tile0; t < desc[i].tile0 + desc[i].tiles; t++)
                BMK_REQUIRE(tmap[t] == (unsigned)i, "q8 matvec multi: tile_map[%d]=%u, expected %d", t, tmap[t], i);
    } else {
        BMK_REQUIRE(nprob <= 0x10000 && next_tile <= n_tiles, "q8 matvec multi: %d problems, %ld tiles in %d workgroups",
                    nprob, next_tile, n_tiles);
        std::vector<long> first((size_t)nprob);
        long acc = 0;
        for (int i = 0; i < nprob; i++) {
            first[i] = acc;
            acc += desc[i].tiles;
        }
        std::vector<unsigned char> seen((size_t)acc, 0);
        long named = 0;
        for (int b = 0; b < n_tiles; b++) {
            if (tmap[b] == BMV_IDLE_TILE) continue;
            const unsigned int pi = tmap[b] >> 16, t = tmap[b] & 0xffffu;
            BMK_REQUIRE(pi < (unsigned)nprob && t < (unsigned)desc[pi].tiles && !seen[first[pi] + t],
                        "q8 matvec multi: tile_map[%d]=0x%08x names no tile left to run", b, tmap[b]);
            seen[first[pi] + t] = 1;
            named++;
        }
        BMK_REQUIRE(named == acc, "q8 matvec multi: the tile map runs %ld of %ld tiles", named, acc);
    }
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
