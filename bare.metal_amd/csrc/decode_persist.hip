/* SPDX-License-Identifier: MPL-2.0
 *
 * decode_persist.hip — every layer of a decode step in one persistent
 * kernel on MI355X: instances of 32 workgroups, each on one XCD, running
 * one or two sequences.
 *
 * The reference runs a decode step as one dispatch per graph node
 * (reference src/baremetal/graph.c:126-226, scheduler.c:712-996): per
 * layer RMSNorm, the q/k/v projections, RoPE, KV store, attention, the
 * o projection, the residual add, RMSNorm, gate/up, SwiGLU, down and the
 * residual add.  At batch 1 on MI355X each such launch is bound by its
 * fixed cost (about 2.5 us from one kernel's end to the next one's first
 * useful load) rather than by its bytes, and at batch 32 still about half
 * of a step is launch cost, so this kernel runs the whole layer stack as
 * five phases per layer inside one launch:
 *   1. RMSNorm(x) and q, k, v (Q8 matvecs of 960 rows at SmolLM2-135M);
 *   2. RoPE, KV append and attention, split into (KV head, key chunk)
 *      pieces that write online-softmax partials (max, sum, P.V);
 *   3. each workgroup merges its share of the attention output from the
 *      partials and hands it over; then the o projection, residual;
 *   4. RMSNorm, gate and up, SwiGLU;
 *   5. down projection, residual.
 * A phase costs a chain of memory round trips rather than bytes, so each
 * one is cut to a single round trip for its inputs.  Vector memory
 * requests of a CU leave in order, and one counter covers a wave's loads and
 * stores, so the order of issue decides what waits for what:
 *   - every staging step (the input vector, the attention partials, the
 *     merged attention output, the q/k/v of a KV head) issues all of its
 *     loads before it waits on any,
 *     with in-bounds addresses for unused lanes so that the compiler can
 *     count them; an attention piece's cached keys and values go first;
 *   - the weights of the next matvec phase are issued right after a
 *     phase's inputs have arrived (o in phase 1, the second RMSNorm in phase
 *     2, gate/up in phase 3 behind the merged output, down in phase 4, the
 *     next layer's q/k/v and
 *     first RMSNorm in phase 5), so they stream in while the phase computes,
 *     into registers of their own (per-phase pass counts P_QKV, P_O, P_GU,
 *     P_DN);
 *   - barriers inside a workgroup order LDS only (an LDS fence), so they
 *     do not wait for those weights;
 *   - a workgroup keeps in registers the rows of the residual stream it
 *     owns (the o and down projections split the rows of x the same way),
 *     so a residual add reads nothing.
 *
 * Instances on one XCD each: MI355X hands workgroups to its 8 XCDs
 * round-robin (b to XCD (b + start) % 8, the start depending on the
 * dispatch).  The grid has 8 x DEC_PERSIST_WGS workgroups (twice that for
 * more than 8 instances); instance g takes the workgroups with b % 8 ==
 * g % 8 in the first or second half, so its working workgroups share one L2,
 * and workgroups of instances past G return at once.  An instance runs NB
 * sequences (one or two) through every phase: each weight block's products
 * with all NB staged vectors, the RMSNorms and residuals per sequence, and
 * NB x NKV x nch attention pieces.  Instances share nothing but the step
 * count and the error flag.
 *
 * No grid barrier: every value one phase hands to another workgroup (x, h,
 * q/k/v, the attention partials) is stored together with the epoch of the
 * phase that wrote it, in one 8-byte store, and a reader loads the values
 * themselves with agent-scope loads (which miss the CU's L1, whose lines may
 * be stale, and read the shared L2) until every one carries the epoch it
 * waits for.  A reader thus proceeds as soon as its own inputs are written,
 * one round trip after the last of them, where a barrier cost a counter
 * update after the writers' stores had completed, a poll, and then the
 * loads (≈6% per step).  Epochs are unique per (step, layer, phase): the
 * step count lives in the exchange buffer, which the host never writes.
 * Reuse of a buffer is safe without barriers: every phase's output depends,
 * through the chain of phases, on every workgroup's previous use of the
 * buffer (a workgroup writes x in phase 5 only after reading all of h, which
 * every workgroup wrote after reading x in phase 4, and so on; the
 * conditions are listed at dec_persist_ok and checked on the host).  The
 * spins are bounded in time: on timeout a workgroup sets
 * DecState.sync_error and leaves, and every other poll gives up once it
 * sees the flag, so the grid always drains.  A working workgroup that finds
 * itself on another XCD than a peer (HW_REG_XCC_ID, gathered per step in
 * the exchange buffer's placement slots) sets the flag before its first
 * wait.  The host reads the flag after the step and reruns a flagged step
 * on the per-phase kernels.
 *
 * Arithmetic: fp32 throughout, the reference's formulas (RMSNorm
 * (x * inv) * w with eps from graph.c:134, rotate-half RoPE, scale
 * 1/sqrt(HD), first-max softmax merge, SiLU x/(1+e^-x)); the Q8 block dot
 * products are those of the other decode kernels (per block sum, times
 * the scale, blocks added in order).  Only the summation orders differ.
 */
#include "bmk.h"
#include "decode_state.h"
#include "q8_common.h"

#include <string.h>

namespace {

using bmk::Blk;
using bmk::block_dot;
using bmk::load_block;

constexpr int PT = 256;              /* threads per workgroup */
constexpr int P_QKV = 4;             /* most row passes of a lane: q/k/v phase */
constexpr int P_O = 2;               /*   o projection */
constexpr int P_GU = 7;              /*   gate/up (two local rows per output) */
constexpr int P_DN = 4;              /*   down projection */
constexpr int P_MAX = 8;
constexpr int XS_MAX = 4096;         /* floats of the staged input vector */
constexpr int XR = 8;                /* elements of the hidden vector h per thread: H <= 2048 */
constexpr int NW = 4;                /* RMSNorm elements per thread: D <= 1024 */
constexpr int QR = 4;                /* elements of the attention output per thread: NH * HD <= 1024 */
constexpr int BUF_FLAGS = 0x00020000; /* word 3 of a raw buffer resource (32-bit data format) */
constexpr int CPOL_SC1 = 16;         /* buffer load cache policy: agent scope (misses the L1) */
constexpr int HD = 64;               /* head size */
constexpr int KCH = 64;              /* keys of one attention sub-chunk (one per lane) */
constexpr int KV_LDS = 2 * 64 * 64;  /* floats of one attention sub-chunk's keys and values in LDS */
constexpr int APR = HD + 2;          /* one partial: max, sum, P.V[HD] */
constexpr int PS_OFF = 1024;         /* attention: the waves' key probabilities in the staged-vector LDS, past q, k, v */
constexpr float SPIN_SECONDS = 0.2f;
constexpr unsigned long long PEEK_TICKS = 1000; /* 10 us at 100 MHz: from then on a wait reads sync_error */
/* LDS of an instance running NB sequences (NB = 1 or 2): the staged input
 * vectors, NB x at most XS_SEQ floats for NB = 2, and the block products
 * of NB vectors; at most 80 KB, so that two instances share a CU */
constexpr int XS_SEQ = 2048;
template <int NB>
struct PLds {
    static constexpr int XS = NB == 1 ? XS_MAX : NB * XS_SEQ;
    static constexpr int RED = P_MAX * PT * NB;
};

/* threadIdx.x, opaque to the compiler: address arithmetic built on it is
 * redone in every phase instead of being hoisted out of the layer loop and
 * held in registers for the whole kernel (that would crowd out the weight
 * stages). */
__device__ __forceinline__ int tid() {
    int t = (int)threadIdx.x;
    asm volatile("" : "+v"(t));
    return t;
}

static_assert(2 * KCH * HD <= KV_LDS, "a sub-chunk's keys and values fit their LDS");
static_assert(4 * HD + 2 * HD <= PS_OFF && PS_OFF + (PT / 64) * KCH <= XS_MAX, "q, k, v and the probabilities share xs");
static_assert(APR % 2 == 0, "partials load as 16-byte pairs of exchanged values");
static_assert(P_QKV <= P_MAX && P_O <= P_MAX && P_GU <= P_MAX && P_DN <= P_MAX, "pass caps");

/* Keeps the compiler from moving instructions across this point: loads
 * issued before it leave before the ones after it (the CU serves them in
 * order). */
__device__ __forceinline__ void issue_order() { __builtin_amdgcn_sched_barrier(0); }

/* Workgroup barrier for LDS data only: loads from global memory in flight
 * stay in flight (__syncthreads would wait for them). */
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

/* DPP lane moves inside rows of 16 lanes (every source lane valid). */
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float lane_value(float v, int lane) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}
constexpr int DPP_XOR1 = 0xB1;        /* quad_perm [1,0,3,2] */
constexpr int DPP_XOR2 = 0x4E;        /* quad_perm [2,3,0,1] */
constexpr int DPP_HALF_MIRROR = 0x141; /* lane i <- 7 - i within 8 */
constexpr int DPP_MIRROR = 0x140;      /* lane i <- 15 - i within 16 */

/* Sum / max over the 64 lanes of a wave (every lane gets it; all lanes active). */
__device__ __forceinline__ float wsum(float v) {
    v += dpp<DPP_XOR1>(v);
    v += dpp<DPP_XOR2>(v);
    v += dpp<DPP_HALF_MIRROR>(v);
    v += dpp<DPP_MIRROR>(v);
    return (lane_value(v, 0) + lane_value(v, 16)) + (lane_value(v, 32) + lane_value(v, 48));
}
__device__ __forceinline__ float wmax(float v) {
    v = fmaxf(v, dpp<DPP_XOR1>(v));
    v = fmaxf(v, dpp<DPP_XOR2>(v));
    v = fmaxf(v, dpp<DPP_HALF_MIRROR>(v));
    v = fmaxf(v, dpp<DPP_MIRROR>(v));
    return fmaxf(fmaxf(lane_value(v, 0), lane_value(v, 16)), fmaxf(lane_value(v, 32), lane_value(v, 48)));
}

/* Sums over the workgroup of NB values per thread (every thread gets them). */
template <int NB>
__device__ __forceinline__ void bsum(float (&v)[NB], float* sh) {
#pragma unroll
    for (int j = 0; j < NB; j++) v[j] = wsum(v[j]);
    lds_barrier(); /* earlier readers of sh are done */
    if ((tid() & 63) == 0)
#pragma unroll
        for (int j = 0; j < NB; j++) sh[j * (PT / 64) + (tid() >> 6)] = v[j];
    lds_barrier();
#pragma unroll
    for (int j = 0; j < NB; j++) {
        float r = 0.f;
#pragma unroll
        for (int i = 0; i < PT / 64; i++) r += sh[j * (PT / 64) + i];
        v[j] = r;
    }
}

/* Values exchanged between phases (see the file comment): the float's bits
 * in the low word, the epoch of the phase that wrote it in the high word,
 * stored and loaded as one 8-byte access at agent scope (the load misses
 * this CU's L1, whose lines may be stale, and reads the XCD's L2). */
typedef unsigned long long xv_t;

__device__ __forceinline__ void put_xv(xv_t* p, float v, unsigned int ep) {
    /* one 8-byte store, single-copy atomic (value and epoch land together).
     * At wavefront scope it compiles to a plain global_store_dwordx2, which
     * lands in the XCD's shared L2 (the L1 does not hold writes), where the
     * readers' agent-scope loads find it; an agent-scope store (sc1) made the
     * step 14% slower. */
    __hip_atomic_store(p, ((xv_t)ep << 32) | __float_as_uint(v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WAVEFRONT);
}
__device__ __forceinline__ xv_t get_xv(const xv_t* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float xv_val(xv_t u) { return __uint_as_float((unsigned int)u); }

/* What a wait needs: the step state (its sync_error), the workgroup's LDS
 * flag `bad` (read by the workgroup after its next barrier) and the longest
 * wait in 100 MHz ticks. */
struct Sync {
    DecState* st;
    int* bad;
    unsigned long long limit;
};

/* Until `ready(k)` holds for every k of every lane of the wave, reloads
 * (reload(k)) the elements not yet ready.  The spin is bounded in time: on
 * timeout it sets DecState.sync_error (1) and *bad and leaves the values as
 * they are; past PEEK_TICKS it also gives up once any workgroup has set
 * sync_error (a timeout elsewhere, or a workgroup on another XCD than its
 * peers), so the whole grid drains soon after the first error. */
template <int N, typename Ready, typename Reload>
__device__ __forceinline__ void poll_xv(Ready&& ready, Reload&& reload, const Sync& sy) {
    auto all_ready = [&] {
        bool ok = true;
#pragma unroll
        for (int k = 0; k < N; k++) ok = ok && ready(k);
        return __all(ok);
    };
    if (all_ready()) return;
    const unsigned long long t0 = __builtin_amdgcn_s_memrealtime(); /* 100 MHz */
    for (;;) {
#pragma unroll
        for (int k = 0; k < N; k++)
            if (!ready(k)) reload(k);
        if (all_ready()) return;
        const unsigned long long dt = __builtin_amdgcn_s_memrealtime() - t0;
        if (dt > sy.limit) {
            __hip_atomic_store(&sy.st->sync_error, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            *sy.bad = 1;
            return;
        }
        /* a wait that ends normally takes a few microseconds: only a longer
         * one reads the flag, so the common poll is one round trip */
        if (dt > PEEK_TICKS && __hip_atomic_load(&sy.st->sync_error, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) {
            *sy.bad = 1;
            return;
        }
    }
}

/* Elements tid + k * PT (clamped to C - 1) of NB exchanged vectors of C
 * values (vector j at x + j * C), once they carry epoch ep: one round of
 * loads, then polls. */
template <int NB, int N>
__device__ __forceinline__ void get_vec(const xv_t* x, int C, unsigned int ep, float (&v)[NB][N], const Sync& sy) {
    xv_t u[NB * N];
    auto addr = [&](int k) { return x + (k / N) * C + min(tid() + (k % N) * PT, C - 1); };
#pragma unroll
    for (int k = 0; k < NB * N; k++) u[k] = get_xv(addr(k));
    poll_xv<NB * N>([&](int k) { return (unsigned int)(u[k] >> 32) == ep; }, [&](int k) { u[k] = get_xv(addr(k)); },
                    sy);
#pragma unroll
    for (int k = 0; k < NB * N; k++) v[k / N][k % N] = xv_val(u[k]);
}

/* One workgroup's share of a matvec phase: output rows [r0, r1) of
 * y = W xs (xs staged in LDS), or for SwiGLU the pairs (gate row j, up row
 * j), j in [r0, r1), interleaved as local rows 2(j-r0) and 2(j-r0)+1.
 * Lane t owns block column t % nb of row slot t / nb (nb <= PT); local row
 * i = pass * slots + slot. */
struct MvShare {
    const unsigned char* w0; /* rows of W (gate for SwiGLU) */
    const unsigned char* w1; /* up rows for SwiGLU */
    int nb, r0, r1, glu;
};

__device__ __forceinline__ int mv_rows(const MvShare& j) { return (j.r1 - j.r0) * (j.glu ? 2 : 1); }

/* Issues the share's block loads (one block per pass) into blk.  Every lane
 * loads: lanes without a row of their own load the share's first block
 * (row 0 of the matrix for an empty share) and their product is dropped. */
template <int NP>
__device__ __forceinline__ void mv_fetch(const MvShare& j, Blk (&blk)[NP]) {
    const int t = tid(), nb = j.nb, slots = PT / nb, slot = t / nb, bc = t - slot * nb;
    const int n = mv_rows(j);
    const size_t row_bytes = (size_t)nb * 36;
#pragma unroll
    for (int p = 0; p < NP; p++) {
        const int i = p * slots + slot;
        const bool own = slot < slots && i < n;
        const int ic = own ? i : 0;
        const unsigned char* w = j.glu ? ((ic & 1) ? j.w1 : j.w0) : j.w0;
        const int r = n > 0 ? j.r0 + (j.glu ? (ic >> 1) : ic) : 0;
        blk[p] = load_block(w + (size_t)r * row_bytes + (size_t)(own ? bc : 0) * 36);
    }
}

/* The block products of the fetched blocks with each of the NB staged
 * vectors (vector j at xs + j * C) into red[j][local row][nb]. */
template <int NB, int NP>
__device__ __forceinline__ void mv_products(int n, int nb, const Blk (&blk)[NP], const float* xs, int C, float* red) {
    const int t = tid(), slots = PT / nb, slot = t / nb, bc = t - slot * nb;
    if (slot < slots) {
#pragma unroll
        for (int j = 0; j < NB; j++) {
            float xv[32];
#pragma unroll
            for (int i = 0; i < 32; i += 4) {
                const float4 v = *(const float4*)&xs[j * C + 32 * bc + i];
                xv[i] = v.x; xv[i + 1] = v.y; xv[i + 2] = v.z; xv[i + 3] = v.w;
            }
#pragma unroll
            for (int p = 0; p < NP; p++) {
                const int i = p * slots + slot;
                if (i < n) red[(j * n + i) * nb + bc] = block_dot(blk[p], xv);
            }
        }
    }
    lds_barrier();
}

/* Sum of local row `row`'s nb block products by the four lanes of a quad:
 * lane j of the quad adds blocks j, j + 4, ..., then the quad's partial
 * sums are added by two DPP steps, so every lane of the quad holds the
 * row's sum.  All four lanes must be active (callers clamp `row`). */
__device__ __forceinline__ float quad_row_sum(const float* red, int row, int nb) {
    const float* rp = red + row * nb;
    float acc = 0.f;
#pragma unroll 4
    for (int k = tid() & 3; k < nb; k += 4) acc += rp[k];
    acc += dpp<DPP_XOR1>(acc);
    acc += dpp<DPP_XOR2>(acc);
    return acc;
}

/* Products of the fetched blocks with the NB staged vectors (each C long),
 * per-row sums (a quad of lanes per row), and the outputs of sequence s,
 * exchanged with epoch ep at y + s * ldy: for SwiGLU y[r0 + o] = silu(gate)
 * * up (gate row 2o in one quad, up row 2o + 1 in the next), else with the
 * residual y[r0 + o] = xres += sum (also stored to plain[s * ldy + r0 + o]
 * when plain is given).  The residual rows (s, o) a workgroup updates are
 * entries e = s * nout + o, entry e in xres[e / 64] of thread 4 (e % 64). */
template <int NB, int NP>
__device__ __forceinline__ void mv_finish(const MvShare& j, const Blk (&blk)[NP], const float* xs, int C, float* red,
                                          xv_t* y, int ldy, unsigned int ep, float (&xres)[NB], float* plain) {
    const int nb = j.nb, nout = j.r1 - j.r0, t = tid(), n = mv_rows(j), tot = NB * nout;
    mv_products<NB>(n, nb, blk, xs, C, red);
    if (j.glu) {
        for (int e0 = 0; e0 < tot; e0 += PT / 8) {
            const int e = min(e0 + (t >> 3), tot - 1), s = e / nout, o = e - s * nout;
            const int row = s * n + min(2 * o + ((t >> 2) & 1), 2 * nout - 1);
            const float sum = quad_row_sum(red, row, nb);
            const float up = dpp<DPP_HALF_MIRROR>(sum); /* lane i of 8 <- 7 - i: the other quad's sum */
            if ((t & 7) == 0 && e0 + (t >> 3) < tot) put_xv(y + s * ldy + j.r0 + o, (sum / (1.0f + expf(-sum))) * up, ep);
        }
    } else {
#pragma unroll
        for (int it = 0; it < NB; it++) {
            if (it * (PT / 4) >= tot) break;
            const int e = it * (PT / 4) + (t >> 2), ec = min(e, tot - 1), s = ec / nout, o = ec - s * nout;
            const float sum = quad_row_sum(red, s * n + o, nb);
            if ((t & 3) == 0 && e < tot) {
                xres[it] += sum;
                put_xv(y + s * ldy + j.r0 + o, xres[it], ep);
                if (plain) plain[s * ldy + j.r0 + o] = xres[it];
            }
        }
    }
}

/* Loads of N elements per thread of a read-only vector of C floats (element
 * threadIdx + k * PT; past the end: element C - 1, masked by the users). */
template <int N>
__device__ __forceinline__ void load_vec(const float* x, int C, float (&v)[N]) {
#pragma unroll
    for (int k = 0; k < N; k++) v[k] = x[min(tid() + k * PT, C - 1)];
}

/* xs[j] = RMSNorm(x_j) * nw from the loaded elements of NB vectors, C <=
 * NW * PT (reference forward.metal:1019-1060: inv = 1/sqrt(mean(x^2) +
 * eps), (x * inv) * w). */
template <int NB>
__device__ __forceinline__ void norm_to_lds(const float (&v)[NB][NW], int C, const float (&nw)[NW], float eps,
                                            float* xs, float* sh) {
    float ss[NB];
#pragma unroll
    for (int j = 0; j < NB; j++) {
        ss[j] = 0.f;
#pragma unroll
        for (int k = 0; k < NW; k++) {
            const float e = tid() + k * PT < C ? v[j][k] : 0.f;
            ss[j] = fmaf(e, e, ss[j]);
        }
    }
    bsum<NB>(ss, sh);
#pragma unroll
    for (int j = 0; j < NB; j++) {
        const float inv = 1.0f / sqrtf(ss[j] / (float)C + eps);
#pragma unroll
        for (int k = 0; k < NW; k++) {
            const int i = tid() + k * PT;
            if (i < C) xs[j * C + i] = (v[j][k] * inv) * nw[k];
        }
    }
    lds_barrier();
}

/* xs[j] = x_j from the loaded elements of NB vectors, C <= N * PT. */
template <int NB, int N>
__device__ __forceinline__ void vec_to_lds(const float (&v)[NB][N], int C, float* xs) {
#pragma unroll
    for (int j = 0; j < NB; j++)
#pragma unroll
        for (int k = 0; k < N; k++) {
            const int i = tid() + k * PT;
            if (i < C) xs[j * C + i] = v[j][k];
        }
    lds_barrier();
}

/* The workgroup's rows of a matrix with R rows: an even split over DEC_PERSIST_WGS. */
__device__ __forceinline__ void share_rows(int R, int w, int& r0, int& r1) {
    r0 = (int)((long)R * w / DEC_PERSIST_WGS);
    r1 = (int)((long)R * (w + 1) / DEC_PERSIST_WGS);
}

/* One attention piece (sequence s of the instance, KV head kh, key chunk c
 * of nch over the keys 0..pos): keys [k0, k1), of which those below lim are
 * in the cache and key pos (if here) is this step's. */
struct Piece {
    int s, kh, c, nch, kv_mul, nq, nraw, k0, k1, lim;
    float* kT; /* the KV head's K cache, [HD/4][MS] float4 */
    float* vc; /* its V cache rows, stride KV */
};

/* Piece w of the instance whose first sequence is b0 (the session's KV
 * cache is [B][L][2][MS * KV]). */
__device__ __forceinline__ Piece make_piece(const DecPersist& a, int layer, int w, int pos, int b0, int nch) {
    Piece p;
    const int per = a.NKV * nch;
    p.s = w / per;
    p.kh = (w - p.s * per) / nch;
    p.c = w - p.s * per - p.kh * nch;
    p.nch = nch;
    p.kv_mul = a.NH / a.NKV;
    p.nq = p.kv_mul * HD;
    p.nraw = p.nq + 2 * HD;
    const int S = pos + 1, cs = (S + nch - 1) / nch;
    p.k0 = p.c * cs;
    p.k1 = min(S, p.k0 + cs);
    p.lim = min(p.k1, pos);
    const size_t slab = (size_t)a.MS * a.KV;
    const size_t sl = (size_t)(b0 + p.s) * a.L + layer; /* this sequence's layer */
    p.kT = a.kvc + sl * 2 * slab + (size_t)p.kh * HD * a.MS;
    p.vc = a.kvc + (sl * 2 + 1) * slab + p.kh * HD;
    return p;
}

/* Keys and values of one attention sub-chunk from the cache, 4 float4 of
 * each per thread on their way to LDS (K as [HD/4][KCH] float4, V as
 * [KCH][HD]); q, k, v of the KV head (raw, [q heads | k | v]). */
constexpr int KV4 = KCH * HD / 4 / PT;
typedef float f4 __attribute__((ext_vector_type(4))); /* plain vector loads and stores (no memcpy) */
struct AttnRegs {
    f4 k[KV4];
    f4 v[KV4];
    float r0, r1;
};

__device__ __forceinline__ void load_kv(const DecPersist& a, const Piece& p, int base, AttnRegs& r) {
    const int t = tid();
#pragma unroll
    for (int j = 0; j < KV4; j++) {
        const int f = t + PT * j;
        const int kkey = base + f % KCH, jj = f / KCH;
        r.k[j] = *(const f4*)(p.kT + ((size_t)jj * a.MS + (kkey < p.lim ? kkey : 0)) * 4);
        const int vkey = base + f / (HD / 4);
        r.v[j] = *(const f4*)(p.vc + (size_t)(vkey < p.lim ? vkey : 0) * a.KV + (f % (HD / 4)) * 4);
    }
}

/* The piece's q, k and v (this step's, exchanged by the previous phase with
 * epoch ep: q at qkv[0, QD), k at qkv[QD, QD + KV), v after it): two
 * elements per thread, polled until they carry ep. */
__device__ __forceinline__ void attn_load(const DecPersist& a, const Piece& p, AttnRegs& r, const xv_t* qkv,
                                          unsigned int ep, const Sync& sy) {
    auto addr = [&](int i) {
        i = min(i, p.nraw - 1);
        return i < p.nq ? qkv + (size_t)p.kh * p.nq + i
                        : i < p.nq + HD ? qkv + a.QD + p.kh * HD + i - p.nq : qkv + a.QD + a.KV + p.kh * HD + i - p.nq - HD;
    };
    xv_t u[2] = {get_xv(addr(tid())), get_xv(addr(tid() + PT))};
    poll_xv<2>([&](int k) { return (unsigned int)(u[k] >> 32) == ep; },
               [&](int k) { u[k] = get_xv(addr(tid() + k * PT)); }, sy);
    r.r0 = xv_val(u[0]);
    r.r1 = xv_val(u[1]);
}

/* The sub-chunk's cached keys and values into LDS. */
__device__ __forceinline__ void put_kv(const Piece& p, int base, const AttnRegs& r, f4* kst, float* vst) {
#pragma unroll
    for (int j = 0; j < KV4; j++) {
        const int f = tid() + PT * j;
        if (base + f % KCH < p.lim) kst[f] = r.k[j];
        const int kk = f / (HD / 4);
        if (base + kk < p.lim) *(f4*)&vst[kk * HD + (f % (HD / 4)) * 4] = r.v[j];
    }
}

/* Attention piece (see Piece) of one layer: RoPE of the group's query heads
 * and of the current key (in registers: lane d of a head's wave pairs with
 * lane d ^ 32; rc, rs = cos, sin of the lane's rotation angle), the KV
 * append by the piece holding pos, then per query head (one wave each) the
 * online softmax over the chunk's keys in sub-chunks of KCH (lane = key for
 * the scores, lane = dimension for P.V, the sub-chunk's values in LDS),
 * written as (max, sum, P.V[HD]) to the partial buffer. */
__device__ __forceinline__ void attn_compute(const DecPersist& a, const Piece& p, int pos, float rc, float rs, AttnRegs& r,
                             float* lds, float* kvs, xv_t* apart, unsigned int ep) {
    const int t = tid(), wave = t >> 6, lane = t & 63;
    const int qk = p.nq + HD; /* roped elements */
    f4* kst = (f4*)kvs;
    float* vst = kvs + KCH * HD;
    {
        const float x0 = r.r0, x1 = r.r1;
        const float y0 = __shfl_xor(x0, 32, 64), y1 = __shfl_xor(x1, 32, 64);
        const float o0 = t >= qk ? x0 : lane < 32 ? x0 * rc - y0 * rs : y0 * rs + x0 * rc;
        const float o1 = t + PT >= qk ? x1 : lane < 32 ? x1 * rc - y1 * rs : y1 * rs + x1 * rc;
        if (t < p.nraw) lds[t] = o0;
        if (t + PT < p.nraw) lds[t + PT] = o1;
        /* this step's key column and value row of the sub-chunk */
        if (pos < p.k0 + KCH && p.k1 == pos + 1) {
            const int kk = pos - p.k0;
            float* row = vst + kk * HD;
            if (t >= p.nq && t < qk) ((float*)&kst[((t - p.nq) >> 2) * KCH + kk])[(t - p.nq) & 3] = o0;
            if (t + PT >= p.nq && t + PT < qk) ((float*)&kst[((t + PT - p.nq) >> 2) * KCH + kk])[(t + PT - p.nq) & 3] = o1;
            if (t >= qk && t < p.nraw) row[t - qk] = x0;
            if (t + PT >= qk && t + PT < p.nraw) row[t + PT - qk] = x1;
        }
    }
    put_kv(p, p.k0, r, kst, vst);
    lds_barrier();
    const float* kc = lds + p.nq;      /* roped current key */
    const float* vr = lds + p.nq + HD; /* current value */
    if (p.k1 == pos + 1 && t < HD) { /* this piece holds position pos: append it */
        p.kT[((size_t)(t >> 2) * a.MS + pos) * 4 + (t & 3)] = kc[t];
        p.vc[(size_t)pos * a.KV + t] = vr[t];
    }
    const float* q = lds + wave * HD;
    float m_run = -INFINITY, l_run = 0.f, acc = 0.f;
    for (int base = p.k0;;) {
        const int n = min(KCH, p.k1 - base);
        if (wave < p.kv_mul) {
            float s = -INFINITY;
            if (lane < n) {
                float s0 = 0.f, s1 = 0.f, s2 = 0.f, s3 = 0.f;
#pragma unroll
                for (int jj = 0; jj < HD / 4; jj++) {
                    const f4 k4 = kst[jj * KCH + lane];
                    s0 = fmaf(q[4 * jj + 0], k4.x, s0);
                    s1 = fmaf(q[4 * jj + 1], k4.y, s1);
                    s2 = fmaf(q[4 * jj + 2], k4.z, s2);
                    s3 = fmaf(q[4 * jj + 3], k4.w, s3);
                }
                s = ((s0 + s1) + (s2 + s3)) * a.scale;
            }
            const float cmax = wmax(s);
            const float pe = lane < n ? expf(s - cmax) : 0.f;
            const float csum = wsum(pe);
            const float m_new = fmaxf(m_run, cmax);
            const float a_old = expf(m_run - m_new), a_new = expf(cmax - m_new);
            /* P.V: the probabilities through LDS (a broadcast read per key)
             * and each batch of 8 keys' reads issued before its FMAs, added
             * in key order; a rolled loop would wait out one LDS round trip
             * per key */
            float* ps = lds + PS_OFF + wave * KCH;
            ps[lane] = pe;
            __builtin_amdgcn_wave_barrier();
            float part = 0.f;
            for (int j0 = 0; j0 < n; j0 += 8) {
                float pp[8], vv[8];
#pragma unroll
                for (int u = 0; u < 8; u++) {
                    const int jk = min(j0 + u, n - 1);
                    pp[u] = ps[jk];
                    vv[u] = vst[jk * HD + lane];
                }
#pragma unroll
                for (int u = 0; u < 8; u++)
                    if (j0 + u < n) part = fmaf(pp[u], vv[u], part);
            }
            __builtin_amdgcn_wave_barrier(); /* ps is rewritten by the next sub-chunk */
            l_run = l_run * a_old + csum * a_new;
            acc = acc * a_old + part * a_new;
            m_run = m_new;
        }
        base += KCH;
        if (base >= p.k1) break;
        lds_barrier(); /* every wave is done with this sub-chunk's keys and values */
        load_kv(a, p, base, r);
        put_kv(p, base, r, kst, vst);
        if (pos >= base && pos < base + KCH && p.k1 == pos + 1 && t < HD) {
            ((float*)&kst[(t >> 2) * KCH + pos - base])[t & 3] = kc[t];
            vst[(pos - base) * HD + t] = vr[t];
        }
        lds_barrier();
    }
    if (wave < p.kv_mul) {
        xv_t* pr = apart + ((size_t)(p.s * a.NH + p.kh * p.kv_mul + wave) * p.nch + p.c) * APR;
        put_xv(pr + 2 + lane, acc, ep);
        if (lane == 0) {
            put_xv(pr, m_run, ep);
            put_xv(pr + 1, l_run, ep);
        }
    }
}

/* The partials of a chunk without keys. */
__device__ __forceinline__ void attn_empty(const DecPersist& a, const Piece& p, xv_t* apart, unsigned int ep) {
    const int wave = tid() >> 6, lane = tid() & 63;
    if (wave < p.kv_mul) {
        xv_t* pr = apart + ((size_t)(p.s * a.NH + p.kh * p.kv_mul + wave) * p.nch + p.c) * APR;
        put_xv(pr + 2 + lane, 0.f, ep);
        if (lane == 0) {
            put_xv(pr, -INFINITY, ep);
            put_xv(pr + 1, 0.f, ep);
        }
    }
}

/* This workgroup's share of the attention output of the NB sequences
 * (elements [o0, o1) of NB x NH*HD, split evenly over the working
 * workgroups), merged from the partials of its nch chunks (exchanged with
 * epoch ep) by wave 0, one element per lane, and exchanged with epoch ep at
 * att: out = sum_c e^(m_c - M) acc_c / sum_c e^(m_c - M) l_c (chunks in
 * order; e^(m_c - M) = 0 for a chunk without keys).  Lanes past the share
 * load element o0's values and store nothing. */
__device__ __forceinline__ void attn_merge_share(const DecPersist& a, int nb, int nch, int w, const xv_t* apart,
                                                 xv_t* att, unsigned int ep, const Sync& sy) {
    if (tid() >= 64) return;
    constexpr int CM = DEC_PERSIST_NCH > DEC_PERSIST_NCH_B ? DEC_PERSIST_NCH : DEC_PERSIST_NCH_B;
    const int tot = nb * a.QD;
    const int o0 = (int)((long)tot * w / DEC_PERSIST_WGS), o1 = (int)((long)tot * (w + 1) / DEC_PERSIST_WGS);
    const int i = o0 + tid(), ic = i < o1 ? i : o0;
    const int sq = ic / a.QD, e = ic - sq * a.QD, h = e / HD, d = e - h * HD;
    const xv_t* pr = apart + (size_t)(sq * a.NH + h) * nch * APR;
    auto addr = [&](int k) {
        const int c = min(k / 3, nch - 1), f = k - 3 * (k / 3);
        return pr + c * APR + (f == 2 ? 2 + d : f);
    };
    xv_t u[3 * CM];
#pragma unroll
    for (int k = 0; k < 3 * CM; k++) u[k] = get_xv(addr(k));
    poll_xv<3 * CM>([&](int k) { return (unsigned int)(u[k] >> 32) == ep; }, [&](int k) { u[k] = get_xv(addr(k)); },
                    sy);
    float M = -INFINITY;
#pragma unroll
    for (int c = 0; c < CM; c++)
        if (c < nch) M = fmaxf(M, xv_val(u[3 * c]));
    float L = 0.f, A = 0.f;
#pragma unroll
    for (int c = 0; c < CM; c++)
        if (c < nch) {
            const float m = xv_val(u[3 * c]);
            const float wc = m == -INFINITY ? 0.f : expf(m - M);
            L = fmaf(wc, xv_val(u[3 * c + 1]), L);
            A = fmaf(wc, xv_val(u[3 * c + 2]), A);
        }
    if (i < o1) put_xv(att + i, A / L, ep);
}

/* HW_REG_XCC_ID bits [3:0] (s_getreg_b32 hwreg(HW_REG_XCC_ID, 0, 4)): the
 * XCD the wave runs on */
constexpr int HWREG_XCC_ID_3_0 = (3 << 11) | (0 << 6) | 20;

/* G instances, each on one XCD (two share an XCD when G > 8, each
 * workgroup of one then sharing a CU with one of the other), each running
 * NB sequences (b0 = g * NB ...) through every layer; the instance's
 * exchanged vectors hold NB rows each. */
template <int NB>
__global__ __launch_bounds__(PT) void k_dec_persist(DecPersist a) {
    /* workgroup b: XCD slot b % 8, then r = b / 8 = 32 h + w: instance g =
     * b % 8 + 8 h (all of whose workgroups share one XCD), working
     * workgroup w of it */
    const int r = (int)(blockIdx.x / 8);
    const int g = (int)(blockIdx.x % 8) + 8 * (r / DEC_PERSIST_WGS);
    if (g >= a.G) return;
    const int w = r % DEC_PERSIST_WGS;
    /* tests only: this workgroup acts as if it ran off its peers' XCD (never
     * workgroup 0, which empties a placement slot below) */
    if (w == a.fault_wg) {
        if (threadIdx.x == 0) __hip_atomic_store(&a.st->sync_error, 2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return;
    }
    __shared__ __attribute__((aligned(16))) float xs[PLds<NB>::XS]; /* staged input vectors, or the attention's q, k, v */
    __shared__ __attribute__((aligned(16))) float red[PLds<NB>::RED];
    __shared__ __attribute__((aligned(16))) float big[KV_LDS]; /* one attention sub-chunk's keys and values */
    __shared__ float sh[NB * (PT / 64)];
    __shared__ int bad; /* a wave of this workgroup timed out waiting for a value */
    DecState* st = a.st;
    const int pos = st->pos;
    const int D = a.D, H = a.H, QD = a.QD, KV = a.KV, QKV = QD + 2 * KV;
    const int nch = NB == 1 ? DEC_PERSIST_NCH : a.nch; /* key chunks per (sequence, KV head) */
    const int b0 = g * NB;                            /* the instance's first sequence */
    const bool has_piece = w < NB * a.NKV * nch;
    /* the instance's exchanged vectors (NB rows each), and the epochs of
     * this step's phases: phase p (1..5) of layer l writes with epoch
     * (steps << 8) + 5 l + p, where steps (advanced by the embedding kernel
     * before every step, never reset; word 0 of the first instance's
     * buffer) is the same for every workgroup of the launch */
    xv_t* exg = a.ex + (size_t)g * a.ex_stride;
    xv_t* xf = exg + DEC_PERSIST_EX_HEAD;
    xv_t* hf = xf + NB * D;
    xv_t* qkvf = hf + NB * H;
    xv_t* apf = qkvf + NB * QKV;
    xv_t* attf = apf + (size_t)NB * a.NH * nch * APR; /* the merged attention output */
    const unsigned int steps = __hip_atomic_load((const unsigned int*)a.ex, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const unsigned int ep0 = steps << 8;
    auto ep = [&](int l, int ph) { return ep0 + (unsigned int)(5 * l + ph); };
    /* The exchange relies on every working workgroup of an instance sharing
     * one XCD's L2 (which one depends on where the dispatch starts).  Each
     * adds its XCD id to this step's placement slot of its instance; one
     * that finds another XCD's bit there flags the step void (sync_error 2)
     * before its first wait (its first-phase outputs may already be
     * written: the step is void either way), the others stop waiting soon
     * after, and the host reruns the step on the per-phase kernels.  The
     * atomic's result is waited for only then, after the whole first
     * phase. */
    const unsigned int xcc_bit = 1u << (__builtin_amdgcn_s_getreg(HWREG_XCC_ID_3_0) & 0xf);
    unsigned int placed = 0;
    if (tid() == 0) placed = atomicOr((unsigned int*)exg + 2 + (steps & 3u), xcc_bit);
    /* the slot of the step after next, emptied now (a device-scope atomic,
     * like the atomicOr's it precedes; this launch ends before that step's
     * kernel starts) */
    if (w == 0 && tid() == 0) atomicExch((unsigned int*)exg + 2 + ((steps + 2u) & 3u), 0u);
    if (tid() == 0) bad = 0;
    const Sync sy = {st, &bad, a.spin_ticks ? a.spin_ticks : (unsigned long long)(SPIN_SECONDS * 1e8f)};

    /* cos, sin of the step's RoPE angle for rotary pair lane % 32 (every
     * sequence is at the same position) */
    float rc, rs;
    {
        const float ang = (float)pos * a.inv_freq[tid() & (HD / 2 - 1)];
        rc = cosf(ang);
        rs = sinf(ang);
    }
    /* the rows of x this workgroup updates (o and down split D the same
     * way): row o of sequence s is entry e = s * (r1 - r0) + o, held in
     * xres[e / 64] of thread 4 (e % 64), the lane that writes it */
    float xres[NB];
    {
        int r0, r1;
        share_rows(D, w, r0, r1);
        const int n = r1 - r0;
#pragma unroll
        for (int it = 0; it < NB; it++) {
            xres[it] = 0.f;
            const int e = it * (PT / 4) + (tid() >> 2);
            if ((tid() & 3) == 0 && e < NB * n)
                xres[it] = a.x[(size_t)(b0 + e / n) * D + r0 + e % n];
        }
    }

    /* the shares of this workgroup in the four matvec phases of a layer */
    auto shares = [&](int l, MvShare& qkv0, MvShare& qkv1, MvShare& qkv2, MvShare& o, MvShare& gu, MvShare& dn) {
        const unsigned char* wl = a.w + (size_t)l * a.layer_bytes;
        const int nbD = D / 32;
        int r0, r1;
        /* q, k, v as one list of QD + 2 KV rows split evenly */
        share_rows(QD + 2 * KV, w, r0, r1);
        qkv0 = {wl + a.off[0], nullptr, nbD, min(r0, QD), min(r1, QD), 0};
        qkv1 = {wl + a.off[1], nullptr, nbD, min(max(r0 - QD, 0), KV), min(max(r1 - QD, 0), KV), 0};
        qkv2 = {wl + a.off[2], nullptr, nbD, min(max(r0 - QD - KV, 0), KV), min(max(r1 - QD - KV, 0), KV), 0};
        share_rows(D, w, r0, r1);
        o = {wl + a.off[3], nullptr, QD / 32, r0, r1, 0};
        share_rows(H, w, r0, r1);
        gu = {wl + a.off[4], wl + a.off[5], nbD, r0, r1, 1};
        share_rows(D, w, r0, r1);
        dn = {wl + a.off[6], nullptr, H / 32, r0, r1, 0};
    };
    /* q, k and v rows of one workgroup come from at most three matrices:
     * their blocks share one register stage, each matrix's rows in order;
     * lanes without a row load the first one (or row 0 of q) */
    auto fetch_qkv = [&](const MvShare& s0, const MvShare& s1, const MvShare& s2, Blk(&blk)[P_QKV]) {
        const int n0 = s0.r1 - s0.r0, n1 = s1.r1 - s1.r0;
        const int t = tid(), nb = s0.nb, slots = PT / nb, slot = t / nb, bc = t - slot * nb;
        const int n = n0 + n1 + (s2.r1 - s2.r0);
        const size_t row_bytes = (size_t)nb * 36;
#pragma unroll
        for (int p = 0; p < P_QKV; p++) {
            const int i = p * slots + slot;
            const bool own = slot < slots && i < n;
            const unsigned char* base = s0.w0;
            int r = 0;
            if (own) {
                if (i < n0) { base = s0.w0; r = s0.r0 + i; }
                else if (i < n0 + n1) { base = s1.w0; r = s1.r0 + i - n0; }
                else { base = s2.w0; r = s2.r0 + i - n0 - n1; }
            }
            blk[p] = load_block(base + (size_t)r * row_bytes + (size_t)(own ? bc : 0) * 36);
        }
    };
    auto finish_qkv = [&](const MvShare& s0, const MvShare& s1, const MvShare& s2, const Blk(&blk)[P_QKV],
                          unsigned int e) {
        const int n0 = s0.r1 - s0.r0, n1 = s1.r1 - s1.r0, n = n0 + n1 + (s2.r1 - s2.r0), tot = NB * n;
        const int nb = s0.nb, o = tid();
        mv_products<NB>(n, nb, blk, xs, D, red);
        for (int e0 = 0; e0 < tot; e0 += PT / 4) {
            const int ei = e0 + (o >> 2), ec = min(ei, tot - 1), sq = ec / n, r = ec - sq * n;
            const float acc = quad_row_sum(red, sq * n + r, nb);
            if ((o & 3) == 0 && ei < tot) {
                xv_t* q = qkvf + sq * QKV;
                if (r < n0) put_xv(q + s0.r0 + r, acc, e);
                else if (r < n0 + n1) put_xv(q + QD + s1.r0 + r - n0, acc, e);
                else put_xv(q + QD + KV + s2.r0 + r - n0 - n1, acc, e);
            }
        }
    };
    auto fetch_norm = [&](const float* nwp, float(&nw)[NW]) { load_vec(nwp, D, nw); };

    Blk bq[P_QKV], bo[P_O], bg[P_GU], bd[P_DN];
    float nw[NW];
    MvShare q0, q1, q2, so, sg, sd;
    shares(0, q0, q1, q2, so, sg, sd);
    fetch_qkv(q0, q1, q2, bq);
    fetch_norm(a.ln1, nw);
    for (int l = 0; l < a.L; l++) {
        /* Two instances per XCD: each CU holds a workgroup of both, and issue
         * goes to the oldest wave first, so the instance dispatched first
         * would run ahead and the step wait for the other.  They take the
         * higher issue priority in turns, one layer each. */
        if (a.G > 8) {
            if ((l + (g >> 3)) & 1) __builtin_amdgcn_s_setprio(1);
            else __builtin_amdgcn_s_setprio(0);
        }
        /* 1. RMSNorm + q, k, v; o's weights stream in behind x.  At the first
         * layer x is the embedding kernel's output (plain). */
        {
            float v[NB][NW];
            if (l == 0) {
#pragma unroll
                for (int j = 0; j < NB; j++) load_vec(a.x + (size_t)(b0 + j) * D, D, v[j]);
            } else {
                get_vec<NB>(xf, D, ep(l - 1, 5), v, sy);
            }
            issue_order();
            mv_fetch(so, bo);
            norm_to_lds<NB>(v, D, nw, a.eps, xs, sh);
        }
        if (bad) return;
        finish_qkv(q0, q1, q2, bq, ep(l, 1));
        /* 2. RoPE + KV append + attention pieces.  The piece's cached keys and
         * values (positions before pos, written by earlier steps) do not
         * depend on this step's q, k, v: their loads go first. */
        {
            /* the placement check, before this workgroup's first wait */
            if (l == 0 && tid() == 0 && (placed & ~xcc_bit)) {
                __hip_atomic_store(&st->sync_error, 2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                bad = 1;
            }
            const Piece pc = make_piece(a, l, w, pos, b0, nch);
            const bool live = has_piece && pc.k0 < pc.k1;
            AttnRegs ar;
            if (live) {
                load_kv(a, pc, pc.k0, ar);
                attn_load(a, pc, ar, qkvf + pc.s * QKV, ep(l, 1), sy);
            }
            issue_order();
            fetch_norm(a.ln2 + (size_t)l * D, nw);
            lds_barrier();
            if (bad) return;
            if (live) attn_compute(a, pc, pos, rc, rs, ar, xs, big, apf, ep(l, 2));
            else if (has_piece) attn_empty(a, pc, apf, ep(l, 2));
        }
        /* 3. merge (this workgroup's share) + o + residual; gate/up weights
         * stream in behind the merged output */
        attn_merge_share(a, NB, nch, w, apf, attf, ep(l, 2), sy);
        {
            float v[NB][QR];
            get_vec<NB>(attf, QD, ep(l, 2), v, sy);
            issue_order();
            mv_fetch(sg, bg);
            vec_to_lds(v, QD, xs);
        }
        if (bad) return;
        mv_finish<NB>(so, bo, xs, QD, red, xf, D, ep(l, 3), xres, nullptr);
        /* 4. RMSNorm + gate, up + SwiGLU; down's weights stream in behind x */
        {
            float v[NB][NW];
            get_vec<NB>(xf, D, ep(l, 3), v, sy);
            issue_order();
            mv_fetch(sd, bd);
            norm_to_lds<NB>(v, D, nw, a.eps, xs, sh);
        }
        if (bad) return;
        mv_finish<NB>(sg, bg, xs, D, red, hf, H, ep(l, 4), xres, nullptr);
        /* 5. down + residual; the next layer's q, k, v and first RMSNorm
         * weights stream in behind h (after the last layer: the last
         * layer's again, unused; no branch, so that h's loads stay first).
         * The last layer also writes x plain, for the LM head. */
        {
            float v[NB][XR];
            get_vec<NB>(hf, H, ep(l, 4), v, sy);
            issue_order();
            const int ln = min(l + 1, a.L - 1);
            shares(ln, q0, q1, q2, so, sg, sd);
            fetch_qkv(q0, q1, q2, bq);
            fetch_norm(a.ln1 + (size_t)ln * D, nw);
            issue_order();
            vec_to_lds(v, H, xs);
        }
        if (bad) return;
        mv_finish<NB>(sd, bd, xs, H, red, xf, D, ep(l, 5), xres, l == a.L - 1 ? a.x + (size_t)b0 * D : nullptr);
    }
}

} // namespace

/* Key chunks per (sequence, KV head) of an instance running NB sequences:
 * enough pieces for the 32 working workgroups, one workgroup each. */
extern "C" int dec_persist_nch(int NKV, int NB) {
    if (NKV <= 0 || NB <= 0) return 0;
    if (NB == 1) return DEC_PERSIST_NCH;
    const int c = DEC_PERSIST_WGS / (NKV * NB);
    return c < DEC_PERSIST_NCH_B ? c : DEC_PERSIST_NCH_B;
}

/* Whether the persistent step can run this shape with NB sequences per
 * instance (NB = 1 or 2): head size 64, every phase's share within its
 * register stage, one output row per thread, the vectors within their LDS
 * stages, and the conditions under which reusing an exchange buffer needs
 * no barrier.  That argument (file comment) is a chain: a buffer is
 * written again only after its writer has read some later phase's output
 * in full, which each of its writers produced only after reading the
 * buffer.  It holds when
 *   (R1) every working workgroup writes rows in phases 1, 3, 4 and 5 (the
 *        q/k/v, o, gate/up and down rows are split evenly over
 *        DEC_PERSIST_WGS, so each needs at least DEC_PERSIST_WGS rows),
 *   (R2) every (sequence, KV head, key chunk) piece has a workgroup, which
 *        writes its partials every step (empty ones too), and
 *   (R3) the merge shares of phase 3 together read every piece's partials,
 *        every workgroup writes a share of the merged output and reads all
 *        of it, and phases 1, 4 and 5 read the whole of x or h in every
 *        workgroup (the kernel's code);
 * (R1) and (R2) are checked here.  Instances share nothing but the step
 * count and the error flag. */
extern "C" int dec_persist_ok_b(int D, int H, int NH, int NKV, int HD_, int MS, int NB) {
    if (NB != 1 && NB != 2) return 0;
    if (HD_ != HD || NKV <= 0 || NH % NKV || NH / NKV > 4 || D % 32 || H % 32 || D > NW * PT || H > XR * PT ||
        NH * HD > QR * PT || MS <= 0)
        return 0;
    const int nch = dec_persist_nch(NKV, NB);
    const int QD = NH * HD, KV = NKV * HD;
    const int xs = NB == 1 ? XS_MAX : NB * XS_SEQ;
    if (NB * QD > xs || NB * D > xs || NB * H > xs) return 0;
    if (QD + 2 * KV < DEC_PERSIST_WGS || D < DEC_PERSIST_WGS || H < DEC_PERSIST_WGS) return 0; /* (R1) */
    if (nch < 1 || NB * NKV * nch > DEC_PERSIST_WGS) return 0;                               /* (R2) */
    auto passes = [](int rows_per_wg, int nb) { return nb > PT ? P_MAX + 1 : (rows_per_wg + PT / nb - 1) / (PT / nb); };
    const int w = DEC_PERSIST_WGS;
    const int qkv = (QD + 2 * KV + w - 1) / w, dr = (D + w - 1) / w, hr = (H + w - 1) / w;
    if (qkv > PT || dr > PT / 4 || hr > PT) return 0; /* residual rows: one per quad of lanes */
    if (passes(qkv, D / 32) > P_QKV) return 0;
    if (passes(dr, QD / 32) > P_O) return 0;
    if (passes(2 * hr, D / 32) > P_GU) return 0;
    if (passes(dr, H / 32) > P_DN) return 0;
    return 1;
}

/* The batch-1 form (one instance, one sequence). */
extern "C" int dec_persist_ok(int D, int H, int NH, int NKV, int HD_, int MS) {
    return dec_persist_ok_b(D, H, NH, NKV, HD_, MS, 1);
}

/* Whether the device fits the kernel's memory-model assumptions: gfx950
 * (MI355X: vector L1 write-through, so a plain store lands in the XCD's
 * L2, and agent-scope loads read that L2), all 256 CUs in one partition,
 * so that workgroups go to the 8 XCDs round-robin and every working
 * workgroup (blockIdx.x % 8 == 0) shares one XCD's L2.  The kernel checks
 * the placement itself at run time (HW_REG_XCC_ID) and flags the step void
 * if it does not hold. */
extern "C" int dec_persist_hw_ok(const char* arch, int cu_count) {
    return arch && strncmp(arch, "gfx950", 6) == 0 && (arch[6] == '\0' || arch[6] == ':') && cu_count == 256;
}

extern "C" int dec_launch_persist(const DecPersist* a, hipStream_t s) {
    BMK_REQUIRE(a->L >= 1 && a->L <= DEC_PERSIST_MAX_L && a->ex, "persistent step: L=%d outside [1, %d] or no exchange buffer",
                a->L, DEC_PERSIST_MAX_L);
    BMK_REQUIRE(a->fault_wg != 0 && a->fault_wg < DEC_PERSIST_WGS, "persistent step: fault workgroup %d outside [1, %d)",
                a->fault_wg, DEC_PERSIST_WGS);
    BMK_REQUIRE(a->G >= 1 && a->G <= 16 && (a->G == 1 || a->ex_stride > 0),
                "persistent step: %d instances (1..16, each with its own exchange rows)", a->G);
    BMK_REQUIRE(a->NB == 1 || (a->nch == dec_persist_nch(a->NKV, a->NB) && a->nch >= 1),
                "persistent step: %d key chunks for %d sequences per instance", a->nch, a->NB);
    BMK_REQUIRE(dec_persist_ok_b(a->D, a->H, a->NH, a->NKV, a->HD, a->MS, a->NB) && a->QD == a->NH * a->HD &&
                    a->KV == a->NKV * a->HD,
                "persistent step: shape D=%d H=%d NH=%d NKV=%d HD=%d with %d sequences per instance not supported", a->D,
                a->H, a->NH, a->NKV, a->HD, a->NB);
    /* up to 8 instances one per XCD, up to 16 two per XCD (each CU then
     * holds a workgroup of both) */
    const dim3 grid(8 * DEC_PERSIST_WGS * (a->G > 8 ? 2 : 1)), block(PT);
    if (a->NB == 1) hipLaunchKernelGGL(k_dec_persist<1>, grid, block, 0, s, *a);
    else hipLaunchKernelGGL(k_dec_persist<2>, grid, block, 0, s, *a);
    BMK_LAUNCH_CHECK();
    return 0;
}
