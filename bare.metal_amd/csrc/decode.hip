/* SPDX-License-Identifier: MPL-2.0
 *
 * decode.hip — the decode-step kernels on gfx950.
 *
 * Two sets, sharing their device code:
 *  1. The kernels the reference's decode scheduler dispatches by name, with
 *     the reference's buffer orders and parameter layouts
 *     (reference src/baremetal/scheduler.c:712-996):
 *       rmsnorm_forward_v2      reference src/kernels/forward.metal:1019-1060
 *       rope_forward            forward.metal:1260-1313
 *       kv_store                forward.metal:1317-1329
 *       attention_forward       forward.metal:1362-1465
 *       add_forward             forward.metal:1332-1340
 *       swiglu_forward          forward.metal:1179-1190
 *       rmsnorm_matmul_forward  forward.metal:1636-1689
 *     plus argmax_f32 (the host-side greedy pick of reference
 *     tools/run.c:56-60 as a kernel: first maximal index wins).
 *  2. The fused kernels of the engine's graph-replayed decode step
 *     (engine.cpp): embedding gather, RMSNorm-prologue Q8 matvecs with
 *     SwiGLU / residual epilogues, rope + KV append + attention, and the
 *     final RMSNorm + LM head + argmax.  They read the position and tokens
 *     from DecState in device memory (decode_state.h).
 *
 * Arithmetic follows the reference kernels term for term where the order is
 * defined (RMSNorm: (x * inv_rms) * w with inv_rms = 1/sqrt(ss/C + eps);
 * RoPE angle (float)pos * inv_freq; SiLU x/(1+exp(-x)); residual a + b);
 * reductions run in fp32 in a fixed order of their own (the reference's
 * order is a fast-math Metal reduction and is not defined).
 */
#include "bmk.h"
#include "decode_state.h"
#include "q8_common.h"
#include "q8_gemm.h"

#include <math.h>
#include <string.h>

namespace {

using namespace bmk;

constexpr int NT = 256;     /* threads per workgroup (4 waves) */
typedef float bmv_f32x4 __attribute__((ext_vector_type(4))); /* fp32 MFMA accumulator tile */
constexpr int ATT_CH = 2048; /* keys per softmax chunk held in LDS */
/* rows in flight per lane in the B = 1 LM head (bandwidth-bound: 113 MB fp32 at 135M): 12 for fp32 rows
 * (256 VGPRs; 0.5% more decode tok/s at 135M than 8, 4 measured 0.8% less), 8 for Q8 and bf16 rows, whose
 * wider per-lane segments would need more than 256 registers at 12 */
constexpr int head_u(int wf) { return wf == 0 ? 12 : 8; }

/* Sum of v over the 256 threads; every thread gets the result.  sh: 4 floats of LDS. */
__device__ __forceinline__ float block_sum(float v, float* sh) {
    v = wave_sum(v);
    const int w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) sh[w] = v;
    __syncthreads();
    float r = (sh[0] + sh[1]) + (sh[2] + sh[3]);
    __syncthreads();
    return r;
}

/* Sum over a workgroup of WT threads (WT/64 waves); every thread gets it. */
template <int WT>
__device__ __forceinline__ float block_sum_t(float v, float* sh) {
    v = wave_sum(v);
    if (WT == 64) return v;
    const int w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) sh[w] = v;
    __syncthreads();
    float r = sh[0];
#pragma unroll
    for (int i = 1; i < WT / 64; i++) r += sh[i];
    __syncthreads();
    return r;
}

__device__ __forceinline__ float block_max(float v, float* sh) {
    v = wave_max(v);
    const int w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) sh[w] = v;
    __syncthreads();
    float r = fmaxf(fmaxf(sh[0], sh[1]), fmaxf(sh[2], sh[3]));
    __syncthreads();
    return r;
}

/* 1/sqrt(mean(x^2) + eps) over C floats (reference forward.metal:1053-1054). */
__device__ __forceinline__ float rms_inv(const float* x, int C, float eps, float* sh) {
    float ss = 0.0f;
    for (int j = threadIdx.x; j < C; j += NT) {
        float v = x[j];
        ss = fmaf(v, v, ss);
    }
    ss = block_sum(ss, sh);
    return 1.0f / sqrtf(ss / (float)C + eps);
}

/* Order-preserving packing of (value, index) for an atomicMax argmax in
 * which the larger value wins and, on equal values, the smaller index: the
 * result of the reference's scan 'if (v[i] > v[best]) best = i' from
 * best = 0 (tools/run.c:56-60, sampler.c:36-39).  That scan treats -0 and
 * +0 as equal, never moves to a NaN, and never moves away from a NaN at
 * index 0; so -0 packs as +0, a NaN packs below every number, and a NaN at
 * index 0 above every number. */
__device__ __forceinline__ unsigned long long argmax_key(float v, int idx) {
    unsigned int u = __float_as_uint(v);
    if (u == 0x80000000u) u = 0u;
    if (v != v) u = idx == 0 ? 0xFFFFFFFFu : 0u;
    else u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return ((unsigned long long)u << 32) | (unsigned long long)(0xFFFFFFFFu - (unsigned int)idx);
}
__device__ __forceinline__ int argmax_key_index(unsigned long long k) {
    return (int)(0xFFFFFFFFu - (unsigned int)(k & 0xFFFFFFFFull));
}

/* Best (value, index) of the workgroup: larger value, then smaller index. */
__device__ __forceinline__ unsigned long long block_argmax_key(unsigned long long k, unsigned long long* sh) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        unsigned long long o = __shfl_xor(k, off, 64);
        k = o > k ? o : k;
    }
    const int w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) sh[w] = k;
    __syncthreads();
    unsigned long long r = sh[0];
#pragma unroll
    for (int i = 1; i < NT / 64; i++) r = sh[i] > r ? sh[i] : r;
    __syncthreads();
    return r;
}

/* ================================================================== */
/* Attention for one query head (one workgroup):
 *   out[d] = sum_t softmax_t(scale * q.k_t) v_t[d],  t < S.
 * Keys t < n_cached come from the cache rows kc/vc (stride KV floats); when
 * cur_k (LDS) is given, key t == n_cached == S-1 is cur_k/cur_v, used from
 * registers so that no pointer ever selects between LDS and global memory.
 * Online softmax over chunks of ATT_CH scores held in LDS.  HD divides 256. */
__device__ void attn_head(const float* qs, const float* kc, const float* vc, int KV, int S, int n_cached,
                          const float* cur_k, const float* cur_v, int HD, float scale, float* sc, float* red,
                          float* sh, float* out) {
    const int t = threadIdx.x;
    const int G = NT / HD, g = t / HD, d = t - g * HD;
    float s_cur = 0.0f, v_cur = 0.0f;
    if (cur_k) {
        float c0 = 0.f, c1 = 0.f;
        for (int e = 0; e < HD; e += 2) {
            c0 = fmaf(qs[e], cur_k[e], c0);
            c1 = fmaf(qs[e + 1], cur_k[e + 1], c1);
        }
        s_cur = (c0 + c1) * scale;
        v_cur = cur_v[d];
    }
    float m_run = -INFINITY, l_run = 0.0f, acc = 0.0f;
    for (int base = 0; base < S; base += ATT_CH) {
        const int n = min(ATT_CH, S - base);
        float lmax = -INFINITY;
        for (int i = t; i < n; i += NT) {
            const int tt = base + i;
            float s;
            if (tt < n_cached) {
                const float* kr = kc + (size_t)tt * KV;
                float s0 = 0.f, s1 = 0.f, s2 = 0.f, s3 = 0.f;
                for (int e = 0; e < HD; e += 4) {
                    float4 kv4;
                    __builtin_memcpy(&kv4, __builtin_assume_aligned(kr + e, 4), 16);
                    s0 = fmaf(qs[e + 0], kv4.x, s0);
                    s1 = fmaf(qs[e + 1], kv4.y, s1);
                    s2 = fmaf(qs[e + 2], kv4.z, s2);
                    s3 = fmaf(qs[e + 3], kv4.w, s3);
                }
                s = ((s0 + s1) + (s2 + s3)) * scale;
            } else {
                s = s_cur;
            }
            sc[i] = s;
            lmax = fmaxf(lmax, s);
        }
        const float cmax = block_max(lmax, sh);
        float lsum = 0.0f;
        for (int i = t; i < n; i += NT) {
            const float p = expf(sc[i] - cmax);
            sc[i] = p;
            lsum += p;
        }
        const float csum = block_sum(lsum, sh); /* its barriers also publish sc[] */
        const float m_new = fmaxf(m_run, cmax);
        const float a_old = expf(m_run - m_new), a_new = expf(cmax - m_new);
        l_run = l_run * a_old + csum * a_new;
        float part = 0.0f;
        const int n_c = min(n, n_cached - base); /* keys of this chunk that are in the cache */
        for (int i = g; i < n_c; i += G) part = fmaf(sc[i], vc[(size_t)(base + i) * KV + d], part);
        if (n_c < n && g == (n_c % G) && n_c >= 0) part = fmaf(sc[n_c], v_cur, part);
        acc = acc * a_old + part * a_new;
        m_run = m_new;
        __syncthreads(); /* sc[] is rewritten by the next chunk */
    }
    red[g * HD + d] = acc;
    __syncthreads();
    if (t < HD) {
        float s = 0.0f;
        for (int k = 0; k < G; k++) s += red[k * HD + t];
        out[t] = s / l_run;
    }
}

/* ================================================================== */
/* Reference-named kernels */

__global__ __launch_bounds__(NT) void k_rmsnorm(const float* __restrict__ x, const float* __restrict__ w,
                                                float* out, int C, float eps) {
    __shared__ float sh[4];
    const float* xr = x + (size_t)blockIdx.x * C;
    float* orow = out + (size_t)blockIdx.x * C;
    const float inv = rms_inv(xr, C, eps, sh);
    for (int j = threadIdx.x; j < C; j += NT) orow[j] = (xr[j] * inv) * w[j];
}

struct RopeTab {
    float inv[DEC_MAX_HD / 2];
};

/* one thread per (head, rotary pair) */
__global__ __launch_bounds__(NT) void k_rope(float* q, float* k, int NH, int NKV, int HD, int pos, RopeTab rt) {
    const int hd2 = HD / 2;
    const int gid = blockIdx.x * NT + threadIdx.x;
    if (gid >= NH * hd2) return;
    const int h = gid / hd2, i = gid - h * hd2;
    const float fr = rt.inv[i];
    const float ang = (float)pos * fr;
    const float c = cosf(ang), s = sinf(ang);
    float* qh = q + h * HD;
    const float q0 = qh[i], q1 = qh[i + hd2];
    qh[i] = q0 * c - q1 * s;
    qh[i + hd2] = q0 * s + q1 * c;
    if (h < NKV) {
        float* kh = k + h * HD;
        const float k0 = kh[i], k1 = kh[i + hd2];
        kh[i] = k0 * c - k1 * s;
        kh[i + hd2] = k0 * s + k1 * c;
    }
}

/* every position of a prompt: one thread per (position s, head h, rotary
 * pair i) of q ([S][NH][HD]) and, for h < NKV, of k ([S][NKV][HD]); the
 * angle is (float)s * inv[i], as k_rope takes it at pos = s */
__global__ __launch_bounds__(NT) void k_rope_seq(float* q, float* k, int S, int NH, int NKV, int HD, RopeTab rt) {
    const int hd2 = HD / 2;
    const long gid = (long)blockIdx.x * NT + threadIdx.x;
    if (gid >= (long)S * NH * hd2) return;
    const int i = (int)(gid % hd2);
    const long sh = gid / hd2;
    const int h = (int)(sh % NH), sp = (int)(sh / NH);
    const float ang = (float)sp * rt.inv[i];
    const float c = cosf(ang), sn = sinf(ang);
    float* qh = q + ((size_t)sp * NH + h) * HD;
    const float q0 = qh[i], q1 = qh[i + hd2];
    qh[i] = q0 * c - q1 * sn;
    qh[i + hd2] = q0 * sn + q1 * c;
    if (h < NKV) {
        float* kh = k + ((size_t)sp * NKV + h) * HD;
        const float k0 = kh[i], k1 = kh[i + hd2];
        kh[i] = k0 * c - k1 * sn;
        kh[i + hd2] = k0 * sn + k1 * c;
    }
}

__global__ __launch_bounds__(NT) void k_kv_store(float* kvc, const float* k, const float* v, int layer, int pos,
                                                 int MS, int KV) {
    const int i = blockIdx.x * NT + threadIdx.x;
    if (i >= KV) return;
    const size_t base = ((size_t)layer * 2 * MS + pos) * KV + i;
    kvc[base] = k[i];
    kvc[base + (size_t)MS * KV] = v[i];
}

__global__ __launch_bounds__(NT) void k_attention(const float* __restrict__ q, const float* __restrict__ kvc,
                                                  float* __restrict__ out, int HD, int KV, int S, int kv_mul,
                                                  int layer, int MS, float scale) {
    __shared__ float qs[256];
    __shared__ float sc[ATT_CH];
    __shared__ float red[NT];
    __shared__ float sh[4];
    const int h = blockIdx.x, kh = h / kv_mul;
    if (threadIdx.x < HD) qs[threadIdx.x] = q[h * HD + threadIdx.x];
    __syncthreads();
    const float* kc = kvc + (size_t)layer * 2 * MS * KV + kh * HD;
    const float* vc = kc + (size_t)MS * KV;
    attn_head(qs, kc, vc, KV, S, S, nullptr, nullptr, HD, scale, sc, red, sh, out + h * HD);
}

__global__ __launch_bounds__(NT) void k_add(const float* a, const float* b, float* out, int n) {
    const int i = blockIdx.x * NT + threadIdx.x;
    if (i < n) out[i] = a[i] + b[i];
}

__global__ __launch_bounds__(NT) void k_swiglu(const float* gate, const float* up, float* out, int n) {
    const int i = blockIdx.x * NT + threadIdx.x;
    if (i < n) out[i] = silu_mul(gate[i], up[i]);
}

/* ================================================================== */
/* LM head: logits[b][r] = sum_j (x[b][j] * inv_b * nw[j]) * W[r][j].
 * fp32 rows: a lane owns 16 consecutive columns (4 dwordx4 loads per row),
 * D/16 lanes cover a row, 256/(D/16) rows per pass, head_u(WF) passes in flight.
 * Q8 rows: a lane owns one 32-column block, as in the Q8 matvec.
 * bf16 rows: a lane owns 32 consecutive columns (4 dwordx4 loads per row),
 * each weight widened to fp32 exactly (bits << 16).
 * With st != NULL the workgroup's best (logit, index) goes into st->key[b]
 * by atomicMax, and the last workgroup to finish turns the keys into
 * tokens, emits them and advances the position. */
/* atomicMax of a workgroup's best key, waited for: the returned value is
 * consumed (into LDS) before the caller's next barrier, so the update has
 * been performed before the workgroup's arrival is counted. */
__device__ __forceinline__ void head_key_max(unsigned long long* key, unsigned long long v, int* sink) {
    const unsigned long long old = atomicMax(key, v);
    if (old == 0xffffffffffffffffull) *sink = 1;
    __atomic_signal_fence(__ATOMIC_SEQ_CST); /* the compiler keeps later accesses after the wait */
}

/* Last workgroup of a head launch (every workgroup calls this after its
 * atomicMax): emit the step's tokens and advance the position.
 *
 * Everything the workgroups of the launch exchange is a device-scope atomic
 * (the per-row argmax keys, the arrival counter), and those are performed
 * at one point for every XCD.  A workgroup's atomicMax results are waited
 * for before its barrier (head_key_max), so they are performed before its
 * arrival is counted; the last arrival reads the keys atomically.  No
 * agent-scope fence is needed: on this multi-XCD part one compiles to a
 * writeback and an invalidate of the whole L2 (buffer_wbl2 / buffer_inv
 * sc1), which in every one of some 900 workgroups cost more than the
 * head's weight stream.  The plain stores of the last workgroup (tokens,
 * position) are read by later kernels, after the launch boundary. */
__device__ void head_finish(const DecHead& a, int& last_wg) {
    const int t = threadIdx.x;
    unsigned int* top = a.arr ? &a.arr->cnt[HEAD_GROUPS][0] : &a.st->done;
    if (a.arr) {
        /* this workgroup's group, then the group's last arrival counts the
         * group once (its keys folded into DecState.key, waited for before
         * the barrier, so before that count) */
        const unsigned int grp = blockIdx.x % HEAD_GROUPS, nwg = gridDim.x;
        const unsigned int n_in = nwg / HEAD_GROUPS + (grp < nwg % HEAD_GROUPS ? 1u : 0u);
        const unsigned int ngrp = nwg < HEAD_GROUPS ? nwg : HEAD_GROUPS;
        if (t == 0) last_wg = atomicAdd(&a.arr->cnt[grp][0], 1u) == n_in - 1u;
        __syncthreads();
        if (!last_wg) return;
        __syncthreads(); /* every thread has read last_wg */
        for (int b = t; b < a.B; b += blockDim.x) {
            const unsigned long long k = atomicExch(&a.arr->key[grp][b], 0ull); /* read and re-arm */
            head_key_max(&a.st->key[b], k, &last_wg);
        }
        __syncthreads();
        if (t == 0) {
            atomicExch(&a.arr->cnt[grp][0], 0u);
            last_wg = atomicAdd(top, 1u) == ngrp - 1u;
        }
    } else if (t == 0) {
        const unsigned int prev = atomicAdd(top, 1u);
        last_wg = (prev == (unsigned int)a.tiles - 1u);
    }
    __syncthreads();
    if (!last_wg) return;
    DecState* st = a.st;
    const int pos = st->pos;
    const bool emit = !st->host_mode && pos >= st->n_prompt - 1;
    for (int b = t; b < a.B; b += blockDim.x) {
        const unsigned long long k = atomicExch(&st->key[b], 0ull); /* read and re-arm */
        const int tok = argmax_key_index(k);
        st->last_token[b] = tok;
        if (emit) a.out_tokens[(size_t)st->n_out * a.B + b] = tok;
    }
    __syncthreads();
    if (t == 0) {
        if (emit) st->n_out = st->n_out + 1;
        atomicExch(top, 0u);
        st->pos = pos + 1;
    }
}

/* Where a workgroup of a head launch folds its best key of batch row b:
 * its group's key (two-level arrival), or DecState.key. */
__device__ __forceinline__ unsigned long long* head_key(const DecHead& a, int b) {
    return a.arr ? &a.arr->key[blockIdx.x % HEAD_GROUPS][b] : &a.st->key[b];
}

/* Weight formats of the LM head rows: fp32, Q8_0 blocks, and two 16-bit
 * formats (bf16, IEEE fp16), each widened exactly to fp32. */
enum { HW_F32 = 0, HW_Q8 = 1, HW_BF16 = 2, HW_F16 = 3 };

template <int WF>
__device__ __forceinline__ int head_lanes(int D) { return WF == HW_F32 ? D / 16 : D / 32; }

/* the two bf16 values of a dword, widened exactly to fp32 */
__device__ __forceinline__ float bf16_lo(unsigned int u) { return __uint_as_float(u << 16); }
__device__ __forceinline__ float bf16_hi(unsigned int u) { return __uint_as_float(u & 0xffff0000u); }
/* the same for the 16-bit formats: bf16, or IEEE fp16 (v_cvt_f32_f16, exact) */
template <int WF>
__device__ __forceinline__ float h16_lo(unsigned int u) {
    return WF == HW_F16 ? (float)__builtin_bit_cast(_Float16, (unsigned short)(u & 0xffffu)) : bf16_lo(u);
}
template <int WF>
__device__ __forceinline__ float h16_hi(unsigned int u) {
    return WF == HW_F16 ? (float)__builtin_bit_cast(_Float16, (unsigned short)(u >> 16)) : bf16_hi(u);
}

template <int WF>
__global__ __launch_bounds__(NT) void k_head(DecHead a) {
    constexpr int HEAD_U = head_u(WF);
    __shared__ float red[NT * HEAD_U];
    __shared__ float sh[4];
    __shared__ unsigned long long shk[NT / 64];
    __shared__ int last_wg;
    const int t = threadIdx.x;
    const int D = a.D;
    const int nseg = head_lanes<WF>(D);
    const int slots = NT / nseg;
    const int rows_per_tile = slots * HEAD_U;
    const int slot = t / nseg, sg = t - slot * nseg;
    const bool lane_on = slot < slots;
    const long row0 = (long)blockIdx.x * rows_per_tile;

    /* issue this tile's weight loads first; they do not depend on x.
     * fp32 and bf16 rows both hold 16 dwords per lane and row in wf */
    float wf[HEAD_U][16];
    Blk wb[HEAD_U];
#pragma unroll
    for (int u = 0; u < HEAD_U; u++) {
        const long r = row0 + slot + (long)u * slots;
        const bool ok = lane_on && r < a.V;
        if (WF == HW_Q8) {
            wb[u] = ok ? load_block(a.wq + ((size_t)r * nseg + sg) * 36) : zero_block();
        } else {
            const float* src = WF == HW_F32 ? a.w + (size_t)r * D + 16 * sg
                                            : (const float*)(a.wh + (size_t)r * D + 32 * sg);
#pragma unroll
            for (int i = 0; i < 16; i += 4) {
                float4 v4 = make_float4(0.f, 0.f, 0.f, 0.f);
                if (ok) __builtin_memcpy(&v4, __builtin_assume_aligned(src + i, 4), 16);
                wf[u][i] = v4.x; wf[u][i + 1] = v4.y; wf[u][i + 2] = v4.z; wf[u][i + 3] = v4.w;
            }
        }
    }

    for (int b = 0; b < a.B; b++) {
        const float* xb = a.x + (size_t)b * D;
        constexpr int SEG = WF == HW_F32 ? 16 : 32;
        float xs[SEG], nw[SEG];
        const bool norm = a.norm_w != nullptr; /* the same for the whole launch */
        if (lane_on) {
#pragma unroll
            for (int i = 0; i < SEG; i += 4) {
                float4 v4, g4 = make_float4(1.f, 1.f, 1.f, 1.f);
                __builtin_memcpy(&v4, __builtin_assume_aligned(xb + SEG * sg + i, 4), 16);
                if (norm) __builtin_memcpy(&g4, __builtin_assume_aligned(a.norm_w + SEG * sg + i, 4), 16);
                xs[i] = v4.x; xs[i + 1] = v4.y; xs[i + 2] = v4.z; xs[i + 3] = v4.w;
                nw[i] = g4.x; nw[i + 1] = g4.y; nw[i + 2] = g4.z; nw[i + 3] = g4.w;
            }
        } else {
#pragma unroll
            for (int i = 0; i < SEG; i++) xs[i] = nw[i] = 0.0f;
        }
        if (norm) {
            /* RMSNorm from registers: the lanes of row slot 0 hold every column once */
            float ss = 0.0f;
            if (lane_on && slot == 0) {
#pragma unroll
                for (int i = 0; i < SEG; i++) ss = fmaf(xs[i], xs[i], ss);
            }
            ss = block_sum(ss, sh);
            const float inv = 1.0f / sqrtf(ss / (float)D + a.eps);
#pragma unroll
            for (int i = 0; i < SEG; i++) xs[i] = (xs[i] * inv) * nw[i];
        }
#pragma unroll
        for (int u = 0; u < HEAD_U; u++) {
            float p;
            if (WF == HW_Q8) {
                p = block_dot(wb[u], xs);
            } else if (WF == HW_F32) {
                float p0 = 0.f, p1 = 0.f, p2 = 0.f, p3 = 0.f;
#pragma unroll
                for (int i = 0; i < 16; i += 4) {
                    p0 = fmaf(xs[i], wf[u][i], p0);
                    p1 = fmaf(xs[i + 1], wf[u][i + 1], p1);
                    p2 = fmaf(xs[i + 2], wf[u][i + 2], p2);
                    p3 = fmaf(xs[i + 3], wf[u][i + 3], p3);
                }
                p = (p0 + p1) + (p2 + p3);
            } else {
                float p0 = 0.f, p1 = 0.f, p2 = 0.f, p3 = 0.f;
#pragma unroll
                for (int i = 0; i < 16; i += 2) {
                    const unsigned int w0 = __float_as_uint(wf[u][i]), w1 = __float_as_uint(wf[u][i + 1]);
                    p0 = fmaf(xs[2 * i], h16_lo<WF>(w0), p0);
                    p1 = fmaf(xs[2 * i + 1], h16_hi<WF>(w0), p1);
                    p2 = fmaf(xs[2 * i + 2], h16_lo<WF>(w1), p2);
                    p3 = fmaf(xs[2 * i + 3], h16_hi<WF>(w1), p3);
                }
                p = (p0 + p1) + (p2 + p3);
            }
            if (lane_on) red[(slot + u * slots) * nseg + sg] = p;
        }
        __syncthreads();
        unsigned long long best = 0ull;
        for (int rl = t; rl < rows_per_tile; rl += NT) {
            const long r = row0 + rl;
            if (r < a.V) {
                const float* rp = red + rl * nseg;
                float acc = 0.0f;
                for (int k = 0; k < nseg; k++) acc += rp[k];
                if (a.bias) acc += a.bias[r];
                a.logits[(size_t)b * a.V + r] = acc;
                const unsigned long long kk = argmax_key(acc, (int)r);
                best = kk > best ? kk : best;
            }
        }
        if (a.st) {
            best = block_argmax_key(best, shk);
            if (t == 0) head_key_max(head_key(a, b), best, &last_wg);
        } else {
            __syncthreads(); /* red[] is rewritten for the next row of the batch */
        }
    }

    if (!a.st) return;
    head_finish(a, last_wg);
}

/* Batched LM head (B >= 2) on fp32 MFMA: a workgroup scores 64 vocabulary
 * rows (16 per wave, each wave over the whole of D) for every batch row;
 * same operand feed as k_dec_bmv (lane: 8 consecutive k of its own row per
 * 32 columns).  Final RMSNorm applied as inv_rms(x[b]) * sum_k x g w.  Row
 * maxima: across the 16 columns of a wave by shuffles, across waves through
 * LDS, then one atomicMax per batch row; the last workgroup emits the
 * tokens (head_finish). */
template <int NBT, int WF, bool XL>
__global__ __launch_bounds__(NT) void k_head_b(DecHead a) {
    __shared__ unsigned long long shk[4][16 * NBT];
    __shared__ int last_wg;
    extern __shared__ float4 xs4[]; /* XL: the batch rows in load order, [kb][bt][half][lane] */
    const int t = threadIdx.x, wave = t >> 6, lane = t & 63;
    const int c = lane & 15, g = lane >> 4;
    const int D = a.D, nkb = D / 32;
    const long r = (long)blockIdx.x * 64 + wave * 16 + c;
    const long rc = r < a.V ? r : (long)a.V - 1;
    const float* xr[NBT];
#pragma unroll
    for (int bt = 0; bt < NBT; bt++) xr[bt] = a.x + (size_t)min(16 * bt + c, a.B - 1) * D + 8 * g;
    const float* nwp = a.norm_w + 8 * g;
    bmv_f32x4 acc[NBT];
    float ss[NBT];
#pragma unroll
    for (int bt = 0; bt < NBT; bt++) {
        acc[bt] = bmv_f32x4{0.f, 0.f, 0.f, 0.f};
        ss[bt] = 0.f;
    }
    /* one K block of operands; the next block's loads are issued before the
     * current block's MFMAs */
    struct Ops {
        float wv[8], s, gv[8], xv[NBT][8];
    };
    auto load_x = [&](int kb, Ops& o) {
#pragma unroll
        for (int bt = 0; bt < NBT; bt++) {
            if (XL) {
                const float4 lo = xs4[((kb * NBT + bt) * 2 + 0) * 64 + lane], hi = xs4[((kb * NBT + bt) * 2 + 1) * 64 + lane];
                o.xv[bt][0] = lo.x; o.xv[bt][1] = lo.y; o.xv[bt][2] = lo.z; o.xv[bt][3] = lo.w;
                o.xv[bt][4] = hi.x; o.xv[bt][5] = hi.y; o.xv[bt][6] = hi.z; o.xv[bt][7] = hi.w;
            } else {
                __builtin_memcpy(&o.xv[bt][0], __builtin_assume_aligned(xr[bt] + 32 * kb, 4), 16);
                __builtin_memcpy(&o.xv[bt][4], __builtin_assume_aligned(xr[bt] + 32 * kb + 4, 4), 16);
            }
        }
    };
    auto load_w = [&](int kb, Ops& o) {
        o.s = 1.0f;
        if (WF == HW_Q8) {
            const unsigned char* blk = a.wq + ((size_t)rc * nkb + kb) * 36;
            unsigned int q0, q1;
            __builtin_memcpy(&o.s, __builtin_assume_aligned(blk, 4), 4);
            __builtin_memcpy(&q0, __builtin_assume_aligned(blk + 4 + 8 * g, 4), 4);
            __builtin_memcpy(&q1, __builtin_assume_aligned(blk + 8 + 8 * g, 4), 4);
#pragma unroll
            for (int i = 0; i < 4; i++) {
                o.wv[i] = q8_byte(q0, i);
                o.wv[4 + i] = q8_byte(q1, i);
            }
        } else if (WF == HW_F32) {
            const float* wp = a.w + (size_t)rc * D + 32 * kb + 8 * g;
            __builtin_memcpy(&o.wv[0], __builtin_assume_aligned(wp, 4), 16);
            __builtin_memcpy(&o.wv[4], __builtin_assume_aligned(wp + 4, 4), 16);
        } else {
            uint4 h4;
            __builtin_memcpy(&h4, __builtin_assume_aligned(a.wh + (size_t)rc * D + 32 * kb + 8 * g, 4), 16);
            o.wv[0] = h16_lo<WF>(h4.x); o.wv[1] = h16_hi<WF>(h4.x);
            o.wv[2] = h16_lo<WF>(h4.y); o.wv[3] = h16_hi<WF>(h4.y);
            o.wv[4] = h16_lo<WF>(h4.z); o.wv[5] = h16_hi<WF>(h4.z);
            o.wv[6] = h16_lo<WF>(h4.w); o.wv[7] = h16_hi<WF>(h4.w);
        }
        __builtin_memcpy(&o.gv[0], __builtin_assume_aligned(nwp + 32 * kb, 4), 16);
        __builtin_memcpy(&o.gv[4], __builtin_assume_aligned(nwp + 32 * kb + 4, 4), 16);
    };
    auto load = [&](int kb, Ops& o) {
        load_w(kb, o);
        load_x(kb, o);
    };
    /* three stages: blocks kb + 1 and kb + 2 in flight during block kb's
     * products (past the last block the loads repeat it, unused) */
    Ops o0, o1, o2;
    if (XL) {
        /* The batch rows, read by every wave at every K block, are staged
         * once per workgroup straight into LDS (global_load_lds, one 1 KB
         * slice per wave instruction: lane l takes row 16 bt + l % 16,
         * columns 32 kb + 8 (l / 16) + 4 half .. +3), while the first two
         * blocks of weights load into registers; each wave streaming all of
         * x from L2 cost 20 of the head's ~51 us at B = 32. */
        for (int j = wave; j < nkb * NBT * 2; j += 4) {
            const int hh = j & 1, bt = (j >> 1) % NBT, kb = (j >> 1) / NBT;
            const float* src = a.x + (size_t)min(16 * bt + c, a.B - 1) * D + 32 * kb + 8 * g + 4 * hh;
            __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)src,
                                             (__attribute__((address_space(3))) void*)&xs4[j * 64], 16, 0, 0);
        }
        load_w(0, o0);
        load_w(min(1, nkb - 1), o1);
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); /* the slices have landed */
        __syncthreads();
        load_x(0, o0);
        load_x(min(1, nkb - 1), o1);
    } else {
        load(0, o0);
        load(min(1, nkb - 1), o1);
    }
    __builtin_amdgcn_sched_barrier(0);
    auto compute = [&](const Ops& cur) {
#pragma unroll
        for (int bt = 0; bt < NBT; bt++) {
            float xv[8];
#pragma unroll
            for (int i = 0; i < 8; i++) {
                ss[bt] = fmaf(cur.xv[bt][i], cur.xv[bt][i], ss[bt]);
                xv[i] = cur.xv[bt][i] * cur.gv[i];
            }
            if (WF == HW_Q8) {
                bmv_f32x4 d = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int i = 0; i < 8; i++) d = __builtin_amdgcn_mfma_f32_16x16x4f32(xv[i], cur.wv[i], d, 0, 0, 0);
#pragma unroll
                for (int v = 0; v < 4; v++) acc[bt][v] = fmaf(cur.s, d[v], acc[bt][v]);
            } else {
#pragma unroll
                for (int i = 0; i < 8; i++)
                    acc[bt] = __builtin_amdgcn_mfma_f32_16x16x4f32(xv[i], cur.wv[i], acc[bt], 0, 0, 0);
            }
        }
    };
    /* the scheduling barriers keep each stage's loads ahead of the products
     * (the compiler would otherwise sink them to their use) */
    for (int kb = 0; kb < nkb; kb += 3) {
        load(min(kb + 2, nkb - 1), o2);
        __builtin_amdgcn_sched_barrier(0);
        compute(o0);
        if (kb + 1 >= nkb) break;
        load(min(kb + 3, nkb - 1), o0);
        __builtin_amdgcn_sched_barrier(0);
        compute(o1);
        if (kb + 2 >= nkb) break;
        load(min(kb + 4, nkb - 1), o1);
        __builtin_amdgcn_sched_barrier(0);
        compute(o2);
    }
#pragma unroll
    for (int bt = 0; bt < NBT; bt++) {
        float sq = ss[bt];
        sq += __shfl_xor(sq, 16);
        sq += __shfl_xor(sq, 32); /* every lane: sum of squares of batch row 16*bt + c */
#pragma unroll
        for (int v = 0; v < 4; v++) {
            const int b = 16 * bt + 4 * g + v;
            const float inv = 1.0f / sqrtf(__shfl(sq, 4 * g + v) / (float)D + a.eps);
            const float val = acc[bt][v] * inv;
            unsigned long long key = 0ull;
            if (r < a.V && b < a.B) {
                a.logits[(size_t)b * a.V + r] = val;
                key = argmax_key(val, (int)r);
            }
#pragma unroll
            for (int off = 1; off < 16; off <<= 1) {
                const unsigned long long o = __shfl_xor(key, off, 64);
                key = o > key ? o : key;
            }
            if (c == 0) shk[wave][b] = key;
        }
    }
    if (!a.st) return;
    __syncthreads();
    for (int b = t; b < a.B; b += NT) {
        unsigned long long best = shk[0][b];
#pragma unroll
        for (int w = 1; w < 4; w++) best = shk[w][b] > best ? shk[w][b] : best;
        head_key_max(head_key(a, b), best, &last_wg);
    }
    __syncthreads();
    head_finish(a, last_wg);
}

/* argmax_f32: first index of the maximum of v[0..n) (reference tools/run.c:56-60). */
__global__ __launch_bounds__(1024) void k_argmax(const float* __restrict__ v, int n, int* out) {
    __shared__ unsigned long long shk[16];
    unsigned long long best = 0ull;
    for (int i = threadIdx.x; i < n; i += 1024) {
        const unsigned long long k = argmax_key(v[i], i);
        best = k > best ? k : best;
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        unsigned long long o = __shfl_xor(best, off, 64);
        best = o > best ? o : best;
    }
    if ((threadIdx.x & 63) == 0) shk[threadIdx.x >> 6] = best;
    __syncthreads();
    if (threadIdx.x == 0) {
        unsigned long long r = shk[0];
        for (int i = 1; i < 16; i++) r = shk[i] > r ? shk[i] : r;
        out[0] = argmax_key_index(r);
    }
}

/* ================================================================== */
/* Fused engine kernels */

/* x[b] = emb[token_b]; token_b from the host, the prompt, or the last argmax. */
__global__ __launch_bounds__(NT) void k_embed(DecEmbed a) {
    __shared__ int tok_s;
    DecState* st = a.st;
    const int b = blockIdx.x, pos = st->pos;
    /* a new step: new epochs for the values the persistent step kernel exchanges */
    if (a.steps && b == 0 && threadIdx.x == 0) *a.steps += 1u;
    if (threadIdx.x == 0) {
        int tok;
        if (st->host_mode) tok = st->host_token[b];
        else if (pos < st->n_prompt) tok = a.prompt[(size_t)b * st->n_prompt + pos];
        else tok = st->last_token[b];
        if (tok < 0 || tok >= a.V) {
            st->bad_token = 1;
            tok = 0;
        }
        st->token[b] = tok;
        tok_s = tok;
    }
    __syncthreads();
    const float* er = a.emb + (size_t)tok_s * a.D;
    float* xr = a.x + (size_t)b * a.D;
    for (int j = threadIdx.x; j < a.D; j += NT) xr[j] = er[j];
}

/* Fused Q8 matvec phase (see DecMv).  WT threads per workgroup; lane t
 * owns block column t % nb of row slot t / nb (nb = C/32 <= WT); U row
 * passes are loaded before any arithmetic.  Small WT and U give many
 * workgroups of few rows: decode matrices are small, and spreading one over
 * hundreds of CUs keeps each CU's share to a single memory round trip. */
template <int WT, int U, int QF>
__device__ __forceinline__ void dec_mv_body(const DecMv& a, float* red, float* sh) {
    typedef QFmt<QF> F;
    const int t = threadIdx.x;
    int mi = 0;
    while (mi + 1 < a.nmat && (int)blockIdx.x >= a.tile0[mi + 1]) mi++;
    const int tile = (int)blockIdx.x - a.tile0[mi];
    const int nb = a.C / 32;
    const int slots = a.slots;
    const int rows_per_tile = slots * U;
    const int slot = t / nb, bc = t - slot * nb;
    const bool lane_on = slot < slots;
    const long row0 = (long)tile * rows_per_tile;
    const size_t row_bytes = (size_t)nb * F::BYTES;
    const bool glu = a.glu != 0;
    const int OC = a.OC[mi];
    const long nrows = glu ? 2L * OC : (long)OC;

    typename F::Block blk[U];
#pragma unroll
    for (int u = 0; u < U; u++) {
        const long lr = row0 + slot + (long)u * slots;
        if (lane_on && lr < nrows) {
            const unsigned char* wm = glu ? a.w[lr & 1] : a.w[mi];
            const long r = glu ? (lr >> 1) : lr;
            blk[u] = F::load(wm + (size_t)r * row_bytes + (size_t)bc * F::BYTES);
        } else {
            blk[u] = F::zero();
        }
    }

    for (int b = 0; b < a.B; b++) {
        /* every global load of this row is issued before the first reduction:
         * the lane's 32 activations, its 32 norm gains and, for the residual
         * epilogue, the old value of the output row the thread will finish */
        const float* xb = a.x + (size_t)b * a.ldx;
        float xs[32], nw[32];
        if (lane_on) {
            const float* xp = xb + 32 * bc;
#pragma unroll
            for (int i = 0; i < 32; i += 4) {
                float4 v4;
                __builtin_memcpy(&v4, __builtin_assume_aligned(xp + i, 4), 16);
                xs[i] = v4.x; xs[i + 1] = v4.y; xs[i + 2] = v4.z; xs[i + 3] = v4.w;
            }
            if (a.norm_w) {
                const float* np = a.norm_w + 32 * bc;
#pragma unroll
                for (int i = 0; i < 32; i += 4) {
                    float4 v4;
                    __builtin_memcpy(&v4, __builtin_assume_aligned(np + i, 4), 16);
                    nw[i] = v4.x; nw[i + 1] = v4.y; nw[i + 2] = v4.z; nw[i + 3] = v4.w;
                }
            }
        } else {
#pragma unroll
            for (int i = 0; i < 32; i++) xs[i] = nw[i] = 0.0f;
        }
        float res0 = 0.0f;
        if (!glu && a.residual && t < rows_per_tile && row0 + t < OC) res0 = a.y[mi][(size_t)b * OC + row0 + t];
        if (a.norm_w) {
            /* the lanes of row slot 0 hold every column exactly once */
            float ss = 0.0f;
            if (lane_on && slot == 0) {
#pragma unroll
                for (int i = 0; i < 32; i++) ss = fmaf(xs[i], xs[i], ss);
            }
            ss = block_sum_t<WT>(ss, sh);
            const float inv = 1.0f / sqrtf(ss / (float)a.C + a.eps);
#pragma unroll
            for (int i = 0; i < 32; i++) xs[i] = (xs[i] * inv) * nw[i];
        }
#pragma unroll
        for (int u = 0; u < U; u++)
            if (lane_on) red[(slot + u * slots) * nb + bc] = block_dot(blk[u], xs);
        __syncthreads();
        if (glu) {
            const int half = rows_per_tile / 2;
            for (int rl = t; rl < half; rl += WT) {
                const long j = (row0 >> 1) + rl;
                if (j < OC) {
                    const float* rg = red + (2 * rl) * nb;
                    const float* ru = rg + nb;
                    float g = 0.0f, u = 0.0f;
                    for (int k = 0; k < nb; k++) {
                        g += rg[k];
                        u += ru[k];
                    }
                    a.y[0][(size_t)b * OC + j] = silu_mul(g, u);
                }
            }
        } else {
            for (int rl = t; rl < rows_per_tile; rl += WT) {
                const long r = row0 + rl;
                if (r >= OC) break;
                const float* rp = red + rl * nb;
                float acc = 0.0f;
                for (int k = 0; k < nb; k++) acc += rp[k];
                float* yp = a.y[mi] + (size_t)b * OC + r;
                if (a.residual) acc = (rl == t ? res0 : *yp) + acc;
                *yp = acc;
            }
        }
        __syncthreads();
    }
}

template <int WT, int U>
__global__ __launch_bounds__(WT) void k_dec_mv(DecMv a) {
    __shared__ float red[WT * U];
    __shared__ float sh[WT / 64];
    dec_mv_body<WT, U, QF_Q8>(a, red, sh);
}

/* The same phase over Q4_0 weights. */
template <int WT, int U>
__global__ __launch_bounds__(WT) void k_dec_mv4(DecMv a) {
    __shared__ float red[WT * U];
    __shared__ float sh[WT / 64];
    dec_mv_body<WT, U, QF_Q4>(a, red, sh);
}

/* Batched fused Q8 matvec (decode with B >= 2) on fp32 MFMA
 * (v_mfma_f32_16x16x4_f32: D[16][16] += A[16][4] x B[4][16]).
 *
 * A workgroup owns 16 output rows of one matrix (a SwiGLU tile: rows
 * j0..j0+7 of gate and of up) for 16*NBT batch rows (blockIdx.y selects
 * them), 16 per MFMA tile.  Its waves take the K blocks round-robin; the partial
 * tiles are summed through LDS in wave order (the same bits at every run).
 * Per K block, lane l (column c = l%16, k group g = l/16) feeds 8 MFMAs with
 * A = x[b0 + c][32kb + 8g + t] (times the norm gain) and B = q[n0 + c][32kb
 * + 8g + t] (t = 0..7): 8 int8 weights of its own row, converted exactly to
 * fp32; the block result D is scaled by the row's block scale, as the
 * reference scales each block's dot product (forward.metal:575-623).
 * RMSNorm: y[b] = inv_rms(x[b]) * sum_k x[b][k] g[k] w[n][k]; the sum of
 * squares rides along with the x loads (each x element is loaded by exactly
 * one lane per batch tile).  D layout: lane l holds rows 4*(l/16)+v (batch
 * rows) of column l%16 (output row). */
constexpr int DBMV_WAVES = 8;              /* waves per workgroup, splitting the K blocks */
constexpr int DBMV_NT = 64 * DBMV_WAVES;

template <int NBT, int QF>
__device__ __forceinline__ void dec_bmv_body(const DecMv& a, bmv_f32x4 (*part)[NBT][64], float (*ssq)[16 * NBT]) {
    constexpr int BYTES = QFmt<QF>::BYTES;
    constexpr int LANE_OFF = QF == QF_Q4 ? 4 : 8; /* bytes of codes per lane and block */
    const int t = threadIdx.x, wave = t >> 6, lane = t & 63;
    const int c = lane & 15, g = lane >> 4;
    int mi = 0;
    while (mi + 1 < a.nmat && (int)blockIdx.x >= a.tile0[mi + 1]) mi++;
    const int tile = (int)blockIdx.x - a.tile0[mi];
    const int b0 = 16 * NBT * (int)blockIdx.y; /* first batch row of this workgroup */
    const bool glu = a.glu != 0;
    const int OC = a.OC[mi];
    const int nb = a.C / 32;
    const size_t row_bytes = (size_t)nb * BYTES;
    /* this lane's weight row (clamped: rows past OC feed outputs never stored) */
    const int row = glu ? tile * 8 + (c & 7) : tile * 16 + c;
    const unsigned char* wrow =
        (glu ? a.w[c >> 3] : a.w[mi]) + (size_t)min(row, OC - 1) * row_bytes + 4 + LANE_OFF * g;
    const float* xr[NBT];
#pragma unroll
    for (int bt = 0; bt < NBT; bt++) xr[bt] = a.x + (size_t)min(b0 + 16 * bt + c, a.B - 1) * a.ldx + 8 * g;
    const float* nwp = a.norm_w ? a.norm_w + 8 * g : nullptr;

    bmv_f32x4 acc[NBT];
    float ss[NBT];
#pragma unroll
    for (int bt = 0; bt < NBT; bt++) {
        acc[bt] = bmv_f32x4{0.f, 0.f, 0.f, 0.f};
        ss[bt] = 0.f;
    }
    for (int kb = wave; kb < nb; kb += DBMV_WAVES) {
        const unsigned char* blk = wrow + (size_t)kb * BYTES;
        float s;
        unsigned int q0, q1 = 0u;
        __builtin_memcpy(&s, __builtin_assume_aligned(blk - 4 - LANE_OFF * g, 4), 4);
        __builtin_memcpy(&q0, __builtin_assume_aligned(blk, 4), 4);
        if (QF == QF_Q8) __builtin_memcpy(&q1, __builtin_assume_aligned(blk + 4, 4), 4);
        float gv[8];
        if (nwp) {
            float4 g0, g1;
            __builtin_memcpy(&g0, __builtin_assume_aligned(nwp + 32 * kb, 4), 16);
            __builtin_memcpy(&g1, __builtin_assume_aligned(nwp + 32 * kb + 4, 4), 16);
            gv[0] = g0.x; gv[1] = g0.y; gv[2] = g0.z; gv[3] = g0.w;
            gv[4] = g1.x; gv[5] = g1.y; gv[6] = g1.z; gv[7] = g1.w;
        }
        float xv[NBT][8];
#pragma unroll
        for (int bt = 0; bt < NBT; bt++) {
            float4 x0, x1;
            __builtin_memcpy(&x0, __builtin_assume_aligned(xr[bt] + 32 * kb, 4), 16);
            __builtin_memcpy(&x1, __builtin_assume_aligned(xr[bt] + 32 * kb + 4, 4), 16);
            xv[bt][0] = x0.x; xv[bt][1] = x0.y; xv[bt][2] = x0.z; xv[bt][3] = x0.w;
            xv[bt][4] = x1.x; xv[bt][5] = x1.y; xv[bt][6] = x1.z; xv[bt][7] = x1.w;
        }
        float wv[8];
        if (QF == QF_Q4) {
#pragma unroll
            for (int i = 0; i < 8; i++) wv[i] = q4_code(q0, i);
        } else {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                wv[i] = q8_byte(q0, i);
                wv[4 + i] = q8_byte(q1, i);
            }
        }
#pragma unroll
        for (int bt = 0; bt < NBT; bt++) {
            if (nwp) {
#pragma unroll
                for (int i = 0; i < 8; i++) {
                    ss[bt] = fmaf(xv[bt][i], xv[bt][i], ss[bt]);
                    xv[bt][i] *= gv[i];
                }
            }
            bmv_f32x4 d = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int i = 0; i < 8; i++) d = __builtin_amdgcn_mfma_f32_16x16x4f32(xv[bt][i], wv[i], d, 0, 0, 0);
#pragma unroll
            for (int v = 0; v < 4; v++) acc[bt][v] = fmaf(s, d[v], acc[bt][v]);
        }
    }
#pragma unroll
    for (int bt = 0; bt < NBT; bt++) {
        part[wave][bt][lane] = acc[bt];
        if (nwp) {
            float v = ss[bt];
            v += __shfl_xor(v, 16);
            v += __shfl_xor(v, 32);
            if (g == 0) ssq[wave][16 * bt + c] = v;
        }
    }
    __syncthreads();
    if (wave != 0) return;
#pragma unroll
    for (int bt = 0; bt < NBT; bt++) {
        bmv_f32x4 y = part[0][bt][lane];
#pragma unroll
        for (int w = 1; w < DBMV_WAVES; w++) y += part[w][bt][lane];
#pragma unroll
        for (int v = 0; v < 4; v++) {
            const int b = b0 + 16 * bt + 4 * g + v;
            float val = y[v];
            if (nwp) {
                const int bi = 4 * g + v + 16 * bt;
                float sq = ssq[0][bi];
#pragma unroll
                for (int w = 1; w < DBMV_WAVES; w++) sq += ssq[w][bi];
                val *= 1.0f / sqrtf(sq / (float)a.C + a.eps);
            }
            if (glu) {
                const float up = __shfl_xor(val, 8);
                const int j = tile * 8 + c;
                if (c < 8 && j < OC && b < a.B) a.y[0][(size_t)b * OC + j] = silu_mul(val, up);
            } else if (row < OC && b < a.B) {
                float* yp = a.y[mi] + (size_t)b * OC + row;
                *yp = a.residual ? *yp + val : val;
            }
        }
    }
}

template <int NBT>
__global__ __launch_bounds__(DBMV_NT) void k_dec_bmv(DecMv a) {
    __shared__ bmv_f32x4 part[DBMV_WAVES][NBT][64];
    __shared__ float ssq[DBMV_WAVES][16 * NBT];
    dec_bmv_body<NBT, QF_Q8>(a, part, ssq);
}

/* The same over Q4_0 weights: a lane's 8 codes of a block are one dword. */
template <int NBT>
__global__ __launch_bounds__(DBMV_NT) void k_dec_bmv4(DecMv a) {
    __shared__ bmv_f32x4 part[DBMV_WAVES][NBT][64];
    __shared__ float ssq[DBMV_WAVES][16 * NBT];
    dec_bmv_body<NBT, QF_Q4>(a, part, ssq);
}

/* Rope + KV append + attention of one decode step; workgroup (h, b) =
 * query head h of sequence b.  The engine's cache holds, per (sequence,
 * layer), K per KV head as [HD/4][MS] float4 (4 dimensions of one
 * position per 16 bytes; lanes scoring consecutive keys read consecutive
 * 16-byte slots, so a wave's load is 1 KB contiguous) and V row-major
 * ([MS][KV]).
 *  - every workgroup of a KV group ropes the group's key itself (same
 *    instructions, same bits) and uses it for the current position; the
 *    group's first query head appends k and v to the cache;
 *  - scores: one key per lane, its HD loads all in flight;
 *  - P.V: 16 key groups x HD/4 float4 columns (coalesced 16-byte loads);
 *  - online softmax over chunks of ATT_CH keys held in LDS.
 * HDT > 0 fixes the head size at compile time (q in registers). */
/* Attention of query head h of sequence b at position pos, given the
 * un-roped q row, the group's un-roped k row and its v row of that
 * position.  Keys before pos come from the cache; append = true writes this
 * position's k and v to the cache (first head of the group), false leaves
 * the cache alone (prefill: every position is already there).  The output
 * row is a.out + out_row * NH * HD. */
template <int HDT>
__device__ __forceinline__ void dec_attn_head(const DecAttn& a, int h, int b, int pos, bool append, int out_row,
                                              const float* qh, const float* kr, const float* vr) {
    constexpr int HDMAX = HDT > 0 ? HDT : DEC_MAX_HD;
    __shared__ float qs[HDMAX];
    __shared__ float ks[HDMAX];
    __shared__ float vs[HDMAX];
    __shared__ float sc[ATT_CH];
    __shared__ float4 red4[NT];
    __shared__ float sh[4];
    const int HD = HDT > 0 ? HDT : a.HD;
    const int HD4 = HD / 4, KG = NT / HD4;
    const int kv_mul = a.NH / a.NKV, kh = h / kv_mul;
    const int t = threadIdx.x;
    if (t < HD / 2) {
        const float fr = a.inv_freq[t];
        const float ang = (float)pos * fr;
        const float c = cosf(ang), s = sinf(ang);
        const float q0 = qh[t], q1 = qh[t + HD / 2];
        qs[t] = q0 * c - q1 * s;
        qs[t + HD / 2] = q0 * s + q1 * c;
        const float k0 = kr[t], k1 = kr[t + HD / 2];
        ks[t] = k0 * c - k1 * s;
        ks[t + HD / 2] = k0 * s + k1 * c;
    }
    if (t < HD) vs[t] = vr[t];
    __syncthreads();
    const size_t slab = (size_t)a.MS * a.KV;
    float* kT = a.kvc + ((size_t)b * a.L + a.layer) * 2 * slab + (size_t)kh * HD * a.MS;
    float* vc = a.kvc + (((size_t)b * a.L + a.layer) * 2 + 1) * slab + kh * HD;
    if (append && h % kv_mul == 0 && t < HD) {
        kT[((size_t)(t >> 2) * a.MS + pos) * 4 + (t & 3)] = ks[t];
        vc[(size_t)pos * a.KV + t] = vs[t];
    }
    float qr[HDT > 0 ? HDT : 1];
    if (HDT > 0) {
#pragma unroll
        for (int e = 0; e < (HDT > 0 ? HDT : 1); e++) qr[e] = qs[e];
    }
    float s_cur;
    {
        float c0 = 0.f, c1 = 0.f;
        for (int e = 0; e < HD; e += 2) {
            c0 = fmaf(qs[e], ks[e], c0);
            c1 = fmaf(qs[e + 1], ks[e + 1], c1);
        }
        s_cur = (c0 + c1) * a.scale;
    }
    const int S = pos + 1, n_cached = pos;
    const int kg = t / HD4, dg = t - kg * HD4;
    float m_run = -INFINITY, l_run = 0.0f;
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int base = 0; base < S; base += ATT_CH) {
        const int n = min(ATT_CH, S - base);
        float lmax = -INFINITY;
        for (int i = t; i < n; i += NT) {
            const int tt = base + i;
            float s;
            if (tt < n_cached) {
                const float* kcol = kT + (size_t)tt * 4;
                const size_t step = (size_t)a.MS * 4;
                float s0 = 0.f, s1 = 0.f, s2 = 0.f, s3 = 0.f;
                if (HDT > 0) {
                    float4 k4[HDT > 0 ? HDT / 4 : 1];
#pragma unroll
                    for (int j = 0; j < (HDT > 0 ? HDT / 4 : 1); j++)
                        __builtin_memcpy(&k4[j], __builtin_assume_aligned(kcol + j * step, 16), 16);
#pragma unroll
                    for (int j = 0; j < (HDT > 0 ? HDT / 4 : 1); j++) {
                        s0 = fmaf(qr[4 * j + 0], k4[j].x, s0);
                        s1 = fmaf(qr[4 * j + 1], k4[j].y, s1);
                        s2 = fmaf(qr[4 * j + 2], k4[j].z, s2);
                        s3 = fmaf(qr[4 * j + 3], k4[j].w, s3);
                    }
                } else {
                    for (int j = 0; j < HD / 4; j++) {
                        float4 k4;
                        __builtin_memcpy(&k4, __builtin_assume_aligned(kcol + j * step, 16), 16);
                        s0 = fmaf(qs[4 * j + 0], k4.x, s0);
                        s1 = fmaf(qs[4 * j + 1], k4.y, s1);
                        s2 = fmaf(qs[4 * j + 2], k4.z, s2);
                        s3 = fmaf(qs[4 * j + 3], k4.w, s3);
                    }
                }
                s = ((s0 + s1) + (s2 + s3)) * a.scale;
            } else {
                s = s_cur;
            }
            sc[i] = s;
            lmax = fmaxf(lmax, s);
        }
        const float cmax = block_max(lmax, sh);
        float lsum = 0.0f;
        for (int i = t; i < n; i += NT) {
            const float p = expf(sc[i] - cmax);
            sc[i] = p;
            lsum += p;
        }
        const float csum = block_sum(lsum, sh); /* its barriers also publish sc[] */
        const float m_new = fmaxf(m_run, cmax);
        const float a_old = expf(m_run - m_new), a_new = expf(cmax - m_new);
        l_run = l_run * a_old + csum * a_new;
        const int n_c = min(n, n_cached - base); /* keys of this chunk that are in the cache */
        float4 part = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll 8
        for (int i = kg; i < n_c; i += KG) {
            float4 v4;
            __builtin_memcpy(&v4, __builtin_assume_aligned(vc + (size_t)(base + i) * a.KV + 4 * dg, 16), 16);
            const float p = sc[i];
            part.x = fmaf(p, v4.x, part.x);
            part.y = fmaf(p, v4.y, part.y);
            part.z = fmaf(p, v4.z, part.z);
            part.w = fmaf(p, v4.w, part.w);
        }
        if (n_c < n && kg == n_c % KG) {
            const float p = sc[n_c];
            part.x = fmaf(p, vs[4 * dg + 0], part.x);
            part.y = fmaf(p, vs[4 * dg + 1], part.y);
            part.z = fmaf(p, vs[4 * dg + 2], part.z);
            part.w = fmaf(p, vs[4 * dg + 3], part.w);
        }
        acc.x = acc.x * a_old + part.x * a_new;
        acc.y = acc.y * a_old + part.y * a_new;
        acc.z = acc.z * a_old + part.z * a_new;
        acc.w = acc.w * a_old + part.w * a_new;
        m_run = m_new;
        __syncthreads(); /* sc[] is rewritten by the next chunk */
    }
    red4[t] = acc;
    __syncthreads();
    if (t < HD) {
        const int c4 = t >> 2, lane = t & 3;
        float sum = 0.0f;
        for (int k = 0; k < KG; k++) {
            const float4 r = red4[k * HD4 + c4];
            sum += lane == 0 ? r.x : lane == 1 ? r.y : lane == 2 ? r.z : r.w;
        }
        a.out[(size_t)out_row * a.NH * HD + h * HD + t] = sum / l_run;
    }
}

/* B = 1 decode attention with the cache loads issued up front.  While the
 * step holds at most ATT_CH keys, lane t loads the K rows of keys t (and
 * t + NT) and the V rows of its first VJ keys in the P.V layout before the
 * RoPE, so those loads overlap the q/k/v reads and the barriers that
 * follow; scores, softmax and P.V then run on registers and LDS, with the
 * same thread assignment and summation order as dec_attn_head (the same
 * bits).  Loads of keys past the cache are not issued.  How far ahead is
 * chosen from the step's length (more registers in flight only where there
 * are keys to fill them); longer steps take dec_attn_head's chunked path. */
template <int HD, int VJ, bool K2>
__device__ __forceinline__ void attn1_body(const DecAttn& a, int h, int b, int pos, const float* qh, const float* kr,
                                           const float* vr) {
    constexpr int HD4 = HD / 4, KG = NT / HD4;
    __shared__ float qs[HD];
    __shared__ float ks[HD];
    __shared__ float vs[HD];
    __shared__ float sc[ATT_CH];
    __shared__ float4 red4[NT];
    __shared__ float sh[4];
    const int kv_mul = a.NH / a.NKV, kh = h / kv_mul;
    const int S = pos + 1, n_cached = pos;
    const int t = threadIdx.x;
    const size_t slab = (size_t)a.MS * a.KV;
    float* kT = a.kvc + ((size_t)b * a.L + a.layer) * 2 * slab + (size_t)kh * HD * a.MS;
    float* vc = a.kvc + (((size_t)b * a.L + a.layer) * 2 + 1) * slab + kh * HD;
    const int kg = t / HD4, dg = t - kg * HD4;
    float4 kp[HD4], kp2[K2 ? HD4 : 1];
    if (t < n_cached) {
        const float* kcol = kT + (size_t)t * 4;
#pragma unroll
        for (int j = 0; j < HD4; j++)
            __builtin_memcpy(&kp[j], __builtin_assume_aligned(kcol + (size_t)j * a.MS * 4, 16), 16);
    }
    if (K2 && t + NT < n_cached) {
        const float* kcol = kT + (size_t)(t + NT) * 4;
#pragma unroll
        for (int j = 0; j < (K2 ? HD4 : 1); j++)
            __builtin_memcpy(&kp2[j], __builtin_assume_aligned(kcol + (size_t)j * a.MS * 4, 16), 16);
    }
    float4 vp[VJ];
#pragma unroll
    for (int j = 0; j < VJ; j++)
        if (kg + KG * j < n_cached)
            __builtin_memcpy(&vp[j], __builtin_assume_aligned(vc + (size_t)(kg + KG * j) * a.KV + 4 * dg, 16), 16);

    if (t < HD / 2) {
        const float fr = a.inv_freq[t];
        const float ang = (float)pos * fr;
        const float c = cosf(ang), sn = sinf(ang);
        const float q0 = qh[t], q1 = qh[t + HD / 2];
        qs[t] = q0 * c - q1 * sn;
        qs[t + HD / 2] = q0 * sn + q1 * c;
        const float k0 = kr[t], k1 = kr[t + HD / 2];
        ks[t] = k0 * c - k1 * sn;
        ks[t + HD / 2] = k0 * sn + k1 * c;
    }
    if (t < HD) vs[t] = vr[t];
    __syncthreads();
    if (h % kv_mul == 0 && t < HD) {
        kT[((size_t)(t >> 2) * a.MS + pos) * 4 + (t & 3)] = ks[t];
        vc[(size_t)pos * a.KV + t] = vs[t];
    }
    float qr[HD];
#pragma unroll
    for (int e = 0; e < HD; e++) qr[e] = qs[e];
    float s_cur;
    {
        float c0 = 0.f, c1 = 0.f;
        for (int e = 0; e < HD; e += 2) {
            c0 = fmaf(qs[e], ks[e], c0);
            c1 = fmaf(qs[e + 1], ks[e + 1], c1);
        }
        s_cur = (c0 + c1) * a.scale;
    }
    auto score = [&](const float4* k4) {
        float s0 = 0.f, s1 = 0.f, s2 = 0.f, s3 = 0.f;
#pragma unroll
        for (int j = 0; j < HD4; j++) {
            s0 = fmaf(qr[4 * j + 0], k4[j].x, s0);
            s1 = fmaf(qr[4 * j + 1], k4[j].y, s1);
            s2 = fmaf(qr[4 * j + 2], k4[j].z, s2);
            s3 = fmaf(qr[4 * j + 3], k4[j].w, s3);
        }
        return ((s0 + s1) + (s2 + s3)) * a.scale;
    };
    float lmax = -INFINITY;
    if (t < S) {
        const float sv = t < n_cached ? score(kp) : s_cur;
        sc[t] = sv;
        lmax = sv;
    }
    int i0 = t + NT;
    if (K2) {
        if (t + NT < S) {
            const float sv = t + NT < n_cached ? score(kp2) : s_cur;
            sc[t + NT] = sv;
            lmax = fmaxf(lmax, sv);
        }
        i0 += NT;
    }
    for (int i = i0; i < S; i += NT) {
        float sv = s_cur;
        if (i < n_cached) {
            float4 k4[HD4];
            const float* kcol = kT + (size_t)i * 4;
#pragma unroll
            for (int j = 0; j < HD4; j++)
                __builtin_memcpy(&k4[j], __builtin_assume_aligned(kcol + (size_t)j * a.MS * 4, 16), 16);
            sv = score(k4);
        }
        sc[i] = sv;
        lmax = fmaxf(lmax, sv);
    }
    const float cmax = block_max(lmax, sh);
    float lsum = 0.0f;
    for (int i = t; i < S; i += NT) {
        const float p = expf(sc[i] - cmax);
        sc[i] = p;
        lsum += p;
    }
    const float csum = block_sum(lsum, sh); /* its barriers also publish sc[] */
    float4 part = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int j = 0; j < VJ; j++) {
        const int i = kg + KG * j;
        if (i < n_cached) {
            const float p = sc[i];
            part.x = fmaf(p, vp[j].x, part.x);
            part.y = fmaf(p, vp[j].y, part.y);
            part.z = fmaf(p, vp[j].z, part.z);
            part.w = fmaf(p, vp[j].w, part.w);
        }
    }
#pragma unroll 8
    for (int i = kg + KG * VJ; i < n_cached; i += KG) {
        float4 v4;
        __builtin_memcpy(&v4, __builtin_assume_aligned(vc + (size_t)i * a.KV + 4 * dg, 16), 16);
        const float p = sc[i];
        part.x = fmaf(p, v4.x, part.x);
        part.y = fmaf(p, v4.y, part.y);
        part.z = fmaf(p, v4.z, part.z);
        part.w = fmaf(p, v4.w, part.w);
    }
    if (kg == n_cached % KG) { /* the current position, from LDS */
        const float p = sc[n_cached];
        part.x = fmaf(p, vs[4 * dg + 0], part.x);
        part.y = fmaf(p, vs[4 * dg + 1], part.y);
        part.z = fmaf(p, vs[4 * dg + 2], part.z);
        part.w = fmaf(p, vs[4 * dg + 3], part.w);
    }
    red4[t] = part;
    __syncthreads();
    if (t < HD) {
        const int c4 = t >> 2, ln = t & 3;
        float sum = 0.0f;
        for (int k = 0; k < KG; k++) {
            const float4 r = red4[k * HD4 + c4];
            sum += ln == 0 ? r.x : ln == 1 ? r.y : ln == 2 ? r.z : r.w;
        }
        a.out[(size_t)b * a.NH * HD + h * HD + t] = sum / csum;
    }
}

template <int HD>
__global__ __launch_bounds__(NT) void k_dec_attn1(DecAttn a) {
    constexpr int KG = NT / (HD / 4);
    const int h = blockIdx.x, b = blockIdx.y;
    const int kh = h / (a.NH / a.NKV);
    const float* qh = a.q + (size_t)b * a.NH * HD + h * HD;
    const float* kr = a.k + (size_t)b * a.KV + kh * HD;
    const float* vr = a.v + (size_t)b * a.KV + kh * HD;
    const int pos = a.st->pos; /* uniform across the workgroup: so are the branches below */
    if (pos + 1 > ATT_CH) dec_attn_head<HD>(a, h, b, pos, true, b, qh, kr, vr);
    else if (pos < 4 * KG) attn1_body<HD, 4, false>(a, h, b, pos, qh, kr, vr);
    else if (pos < NT) attn1_body<HD, NT / KG, false>(a, h, b, pos, qh, kr, vr);
    else attn1_body<HD, (3 * NT / 2) / KG, true>(a, h, b, pos, qh, kr, vr);
}

template <int HDT>
__global__ __launch_bounds__(NT) void k_dec_attn(DecAttn a) {
    const int HD = HDT > 0 ? HDT : a.HD;
    const int h = blockIdx.x, b = blockIdx.y;
    const int kh = h / (a.NH / a.NKV);
    dec_attn_head<HDT>(a, h, b, a.st->pos, true, b, a.q + (size_t)b * a.NH * HD + h * HD, a.k + (size_t)b * a.KV + kh * HD,
                       a.v + (size_t)b * a.KV + kh * HD);
}


/* Decode attention of one KV-head group: workgroup (KV head kh, sequence b)
 * serves all kv_mul query heads of the group, so each cached key and value
 * row is read once for all of them (GQA).  Its AG_WAVES waves split the
 * positions 0..pos into contiguous ranges; a wave walks its range in chunks
 * of 64 keys:
 *  - scores: lane = key, the key's HD/4 float4 loads issued together (the
 *    [HD/4][MS] K layout makes a wave's load 1 KB contiguous), one dot
 *    product per query head;
 *  - online softmax per head with wave reductions;
 *  - P.V: lane = (key group, float4 column), all of its value loads issued
 *    together, the weights p read back from the wave's LDS row.
 * The waves' (max, sum, partial output) are merged in wave order through
 * LDS.  Thread 0..HD/2 ropes the group's queries and the new key; the new
 * key and value are appended to the cache and used from LDS at position pos. */
constexpr int AG_WAVES = 8;

template <int HD, int KVM>
__global__ __launch_bounds__(64 * AG_WAVES) void k_dec_attn_g(DecAttn a) {
    constexpr int W = AG_WAVES;
    constexpr int AG_MAXM = KVM; /* query heads per KV head (compile time: registers, not scratch) */
    constexpr int HD4 = HD / 4, KGW = 64 / HD4; /* P.V: key groups per wave */
    __shared__ float qs[AG_MAXM][HD];
    __shared__ float kcur[HD];
    __shared__ float vcur[HD];
    __shared__ float ps[W][AG_MAXM][64];
    __shared__ float4 po[W][AG_MAXM][HD4];
    __shared__ float pm[W][AG_MAXM];
    __shared__ float pl[W][AG_MAXM];
    const int kh = blockIdx.x, b = blockIdx.y;
    constexpr int kv_mul = KVM;
    const int t = threadIdx.x, wave = t >> 6, lane = t & 63;
    const int pos = a.st->pos, S = pos + 1;
    if (t < HD / 2) {
        const float fr = a.inv_freq[t];
        const float ang = (float)pos * fr;
        const float c = cosf(ang), sn = sinf(ang);
        for (int j = 0; j < kv_mul; j++) {
            const float* qh = a.q + (size_t)b * a.NH * HD + (size_t)(kh * kv_mul + j) * HD;
            const float q0 = qh[t], q1 = qh[t + HD / 2];
            qs[j][t] = q0 * c - q1 * sn;
            qs[j][t + HD / 2] = q0 * sn + q1 * c;
        }
        const float* kr = a.k + (size_t)b * a.KV + kh * HD;
        const float k0v = kr[t], k1v = kr[t + HD / 2];
        kcur[t] = k0v * c - k1v * sn;
        kcur[t + HD / 2] = k0v * sn + k1v * c;
    }
    if (t < HD) vcur[t] = a.v[(size_t)b * a.KV + kh * HD + t];
    __syncthreads();
    const size_t slab = (size_t)a.MS * a.KV;
    float* kT = a.kvc + ((size_t)b * a.L + a.layer) * 2 * slab + (size_t)kh * HD * a.MS;
    float* vc = a.kvc + (((size_t)b * a.L + a.layer) * 2 + 1) * slab + kh * HD;
    if (t < HD) {
        kT[((size_t)(t >> 2) * a.MS + pos) * 4 + (t & 3)] = kcur[t];
        vc[(size_t)pos * a.KV + t] = vcur[t];
    }
    const int per = (S + W - 1) / W;
    const int w0 = wave * per, w1 = min(S, w0 + per);
    float m_run[AG_MAXM], l_run[AG_MAXM];
    float4 acc[AG_MAXM];
#pragma unroll
    for (int j = 0; j < AG_MAXM; j++) {
        m_run[j] = -INFINITY;
        l_run[j] = 0.0f;
        acc[j] = make_float4(0.f, 0.f, 0.f, 0.f);
    }
    const int kg = lane / HD4, dg = lane % HD4;
    const size_t kstep = (size_t)a.MS * 4;
    for (int c0 = w0; c0 < w1; c0 += 64) {
        const int n = min(64, w1 - c0);
        const int key = c0 + lane;
        const bool valid = lane < n;
        float4 k4[HD4];
        if (valid && key < pos) {
#pragma unroll
            for (int e = 0; e < HD4; e++)
                __builtin_memcpy(&k4[e], __builtin_assume_aligned(kT + (size_t)key * 4 + e * kstep, 16), 16);
        } else {
#pragma unroll
            for (int e = 0; e < HD4; e++) k4[e] = make_float4(kcur[4 * e], kcur[4 * e + 1], kcur[4 * e + 2], kcur[4 * e + 3]);
        }
#pragma unroll
        for (int j = 0; j < AG_MAXM; j++) {
            float s0 = 0.f, s1 = 0.f, s2 = 0.f, s3 = 0.f;
#pragma unroll
            for (int e = 0; e < HD4; e++) {
                s0 = fmaf(qs[j][4 * e + 0], k4[e].x, s0);
                s1 = fmaf(qs[j][4 * e + 1], k4[e].y, s1);
                s2 = fmaf(qs[j][4 * e + 2], k4[e].z, s2);
                s3 = fmaf(qs[j][4 * e + 3], k4[e].w, s3);
            }
            const float sc = valid ? ((s0 + s1) + (s2 + s3)) * a.scale : -INFINITY;
            const float mn = fmaxf(m_run[j], wave_max(sc));
            const float p = valid ? expf(sc - mn) : 0.0f;
            const float alpha = expf(m_run[j] - mn);
            l_run[j] = l_run[j] * alpha + wave_sum(p);
            acc[j].x *= alpha;
            acc[j].y *= alpha;
            acc[j].z *= alpha;
            acc[j].w *= alpha;
            m_run[j] = mn;
            ps[wave][j][lane] = p;
        }
        __builtin_amdgcn_wave_barrier();
        /* P.V over this lane's 64/KGW key slots, in two halves (half the value
         * registers live at a time), each half's loads issued together */
        constexpr int R = 64 / KGW, RH = R > 1 ? R / 2 : 1;
#pragma unroll
        for (int h0 = 0; h0 < R; h0 += RH) {
            float4 v4[RH];
#pragma unroll
            for (int r = 0; r < RH; r++) {
                const int i = kg + (h0 + r) * KGW;
                if (i < n && c0 + i < pos)
                    __builtin_memcpy(&v4[r], __builtin_assume_aligned(vc + (size_t)(c0 + i) * a.KV + 4 * dg, 16), 16);
                else
                    v4[r] = make_float4(vcur[4 * dg], vcur[4 * dg + 1], vcur[4 * dg + 2], vcur[4 * dg + 3]);
            }
#pragma unroll
            for (int j = 0; j < AG_MAXM; j++) {
#pragma unroll
                for (int r = 0; r < RH; r++) {
                    const int i = kg + (h0 + r) * KGW;
                    const float p = i < n ? ps[wave][j][i] : 0.0f;
                    acc[j].x = fmaf(p, v4[r].x, acc[j].x);
                    acc[j].y = fmaf(p, v4[r].y, acc[j].y);
                    acc[j].z = fmaf(p, v4[r].z, acc[j].z);
                    acc[j].w = fmaf(p, v4[r].w, acc[j].w);
                }
            }
        }
        __builtin_amdgcn_wave_barrier(); /* ps is rewritten by the next chunk */
    }
#pragma unroll
    for (int j = 0; j < AG_MAXM; j++) {
#pragma unroll
        for (int off = HD4; off < 64; off <<= 1) {
            acc[j].x += __shfl_xor(acc[j].x, off);
            acc[j].y += __shfl_xor(acc[j].y, off);
            acc[j].z += __shfl_xor(acc[j].z, off);
            acc[j].w += __shfl_xor(acc[j].w, off);
        }
        if (lane < HD4) po[wave][j][lane] = acc[j];
        if (lane == 0) {
            pm[wave][j] = m_run[j];
            pl[wave][j] = l_run[j];
        }
    }
    __syncthreads();
    for (int u = t; u < kv_mul * HD; u += 64 * W) {
        const int j = u / HD, d = u - j * HD;
        float M = -INFINITY;
        for (int w = 0; w < W; w++) M = fmaxf(M, pm[w][j]);
        float num = 0.0f, den = 0.0f;
        for (int w = 0; w < W; w++) {
            if (pm[w][j] == -INFINITY) continue;
            const float f = expf(pm[w][j] - M);
            const float4 o = po[w][j][d >> 2];
            const int c = d & 3;
            den = fmaf(f, pl[w][j], den);
            num = fmaf(f, c == 0 ? o.x : c == 1 ? o.y : c == 2 ? o.z : o.w, num);
        }
        a.out[(size_t)b * a.NH * HD + (size_t)(kh * kv_mul + j) * HD + d] = num / den;
    }
}

/* ------------------------------------------------------------------ */
/* Prefill (bm_forward on a whole prompt at position 0, batch 1): every
 * prompt position at once, the projections on the bf16-MFMA GEMMs of
 * pf_gemm.hip, as the reference's prefill graph runs them on its BT > 1 Q8
 * path (graph.c:273-381, scheduler.c:1015-1332).  The GEMMs' activations
 * are bf16 in MFMA fragment order (frag_index): the RMSNorm and the
 * attention write them so. */

/* x[p] = emb[tok[p]], and the first layer's RMSNorm operand as the q/k/v
 * GEMM takes it (pf_gemm.h): an = bf16(x * g) in fragment order (columns
 * past D zero) and the row's sum of squares in slot 0 of ss (the other
 * ss_tiles - 1 slots zero).  With rope given, also position p's (cos, sin)
 * per rotary pair, rope[p][HD/2][2] (the angle (float)p * inv_freq[t] as
 * k_pf_kv takes it), for the q/k/v GEMM epilogue that rotates k. */
__global__ __launch_bounds__(NT) void k_pf_embed(const int* __restrict__ tok, const float* __restrict__ emb,
                                                 float* __restrict__ x, int D, const float* __restrict__ g,
                                                 unsigned short* __restrict__ an, float* __restrict__ ss_out,
                                                 int ss_tiles, int ss_ld, DecAttn ra, float* __restrict__ rope) {
    __shared__ float sh[4];
    const int p = blockIdx.x;
    if (rope) {
        const int half = ra.HD / 2;
        for (int i = threadIdx.x; i < half; i += NT) {
            const float ang = (float)p * ra.inv_freq[i];
            rope[((size_t)p * half + i) * 2] = cosf(ang);
            rope[((size_t)p * half + i) * 2 + 1] = sinf(ang);
        }
    }
    const float* er = emb + (size_t)tok[p] * D;
    float* xr = x + (size_t)p * D;
    float ss = 0.0f;
    for (int j = threadIdx.x; j < D; j += NT) {
        const float v = er[j];
        xr[j] = v;
        ss = fmaf(v, v, ss);
    }
    ss = block_sum(ss, sh);
    if (threadIdx.x < ss_tiles) ss_out[(size_t)threadIdx.x * ss_ld + p] = threadIdx.x == 0 ? ss : 0.0f;
    const int nks = (D + 63) / 64;
    for (int c = threadIdx.x; c < 8 * nks; c += NT) {
        unsigned int w[4] = {0u, 0u, 0u, 0u};
        if (8 * c < D)
#pragma unroll
            for (int e = 0; e < 4; e++)
                w[e] = (unsigned int)bf16_bits(er[8 * c + 2 * e] * g[8 * c + 2 * e]) |
                       ((unsigned int)bf16_bits(er[8 * c + 2 * e + 1] * g[8 * c + 2 * e + 1]) << 16);
        *(uint4*)(an + frag_index(p, 8 * c, nks)) = make_uint4(w[0], w[1], w[2], w[3]);
    }
}

/* RoPE of every position's k and the cache append of k and v (layer a.layer,
 * sequence 0): workgroup p, thread (KV head, rotary pair). */
__global__ __launch_bounds__(NT) void k_pf_kv(DecAttn a, const float* __restrict__ k, const float* __restrict__ v) {
    const int p = blockIdx.x;
    const int HD = a.HD, half = HD / 2;
    const size_t slab = (size_t)a.MS * a.KV;
    float* kc = a.kvc + (size_t)a.layer * 2 * slab;
    float* vc = kc + slab;
    for (int i = threadIdx.x; i < a.NKV * half; i += NT) {
        const int kh = i / half, t = i - kh * half;
        const float ang = (float)p * a.inv_freq[t];
        const float c = cosf(ang), sn = sinf(ang);
        const size_t kr = (size_t)p * a.KV + kh * HD;
        const float k0 = k[kr + t], k1 = k[kr + t + half];
        float* kT = kc + (size_t)kh * HD * a.MS;
        kT[((size_t)(t >> 2) * a.MS + p) * 4 + (t & 3)] = k0 * c - k1 * sn;
        const int t2 = t + half;
        kT[((size_t)(t2 >> 2) * a.MS + p) * 4 + (t2 & 3)] = k0 * sn + k1 * c;
    }
    for (int i = threadIdx.x; i < a.KV; i += NT) vc[(size_t)p * a.KV + i] = v[(size_t)p * a.KV + i];
}

/* Causal attention of every prompt position: workgroup (query head h,
 * position p) over keys 0..p, the cache already holding all of them. */
template <int HDT>
__global__ __launch_bounds__(NT) void k_pf_attn(DecAttn a, const float* __restrict__ q, const float* __restrict__ k,
                                                const float* __restrict__ v) {
    const int HD = HDT > 0 ? HDT : a.HD;
    const int h = blockIdx.x, p = blockIdx.y;
    const int kh = h / (a.NH / a.NKV);
    dec_attn_head<HDT>(a, h, 0, p, false, p, q + (size_t)p * a.NH * HD + h * HD, k + (size_t)p * a.KV + kh * HD,
                       v + (size_t)p * a.KV + kh * HD);
}

/* Causal attention of a block of PQB = 16 consecutive prompt positions of
 * one query head, head size 64: softmax(q.k * scale) over keys 0..p, times
 * V, on fp32 MFMA (v_mfma_f32_16x16x4f32).  Two sources share the kernel:
 *  - PF_ENGINE: the engine's prefill.  q rows are un-roped ([n][NH*HD]; the
 *    kernel applies RoPE at each position as dec_attn_head does), K and V
 *    come from the KV cache of layer a.layer (K per KV head as
 *    [HD/4][MS] float4, V row-major [MS][KV]), the output is bf16 (the
 *    o-projection's operand).
 *  - PF_FLAT: the reference's prefill attention ABI (forward.metal:1904-2114):
 *    Q roped [S][NH][HD], K and V [S][NKV][HD], fp32 output [S][NH][HD].
 * Keys are staged through LDS in chunks of PKC: K row-major [key][dim],
 * V transposed [dim][key] (rows padded by 4 floats, so the 16 rows a wave
 * reads at once fall in different banks).  The chunk is cut into 16-key
 * sub-blocks dealt round-robin to the waves; per sub-block a wave forms
 *   S^T (16 keys x 16 queries) = K_sb Q^T   (16 MFMAs over the 64 dims),
 * updates a per-query online softmax, and accumulates
 *   O^T (64 dims x 16 queries) += V_sb^T P^T (16 MFMAs).
 * The MFMA sums run over any order of their index, so both products use a
 * permuted one: in S^T, step s of lane group g (= lane/16) takes dimension
 * 16g + s (a lane reads 16 consecutive dims of its key); in O^T, step s of
 * lane group g takes key 4g + s, which is exactly the key whose score that
 * lane holds in element s of its S^T fragment, so P^T goes from the score
 * registers to the next MFMA with no data movement.  Each wave's (max,
 * sum, O^T) is merged across waves through LDS at the end.  Keys at or
 * past n are staged as zeros, masked keys score -inf.  The summation order
 * differs from the one-query kernels; the mathematics is the same. */
constexpr int PQB = 16;  /* prompt positions per workgroup */
#ifndef PF_KCHUNK
#define PF_KCHUNK 128
#endif
#ifndef PF_WAVES
#define PF_WAVES 8
#endif
constexpr int PKC = PF_KCHUNK; /* keys per LDS chunk: one 16-key sub-block per wave and chunk */
constexpr int PNW = PF_WAVES;  /* waves per workgroup: 8 (two per SIMD, one's softmax beside the other's
                                  products) 15.4 us per layer at 512 tokens, 4 waves 18.3 us, 2 waves 27 */
static_assert(PKC == 16 * PNW, "one 16-key sub-block per wave and chunk");
constexpr int PNT = 64 * PNW;
enum { PF_ENGINE = 0, PF_FLAT = 1 };

struct PfFlat {
    const float* Q;
    const float* K;
    const float* V;
    float* out;
    float scale;
    int NH, S, NKV, kv_mul;
};

template <int MODE>
__device__ __forceinline__ void pf_attn_block(const DecAttn& a, const PfFlat& f, const float* __restrict__ q,
                                              unsigned short* __restrict__ out16, int n, int q_roped) {
    constexpr int HD = 64, HD4 = HD / 4;
    constexpr int LDK = HD + 4, LDVT = PKC + 4;
    constexpr int NSB = PKC / 16; /* sub-blocks per chunk */
    __shared__ float Ks[PKC * LDK];   /* [key][dim] */
    __shared__ float Vt[HD * LDVT];   /* [dim][key] */
    __shared__ float Qs[PQB * HD];    /* roped q of the block */
    __shared__ float Ms[PNW * PQB], Ls[PNW * PQB];
    const int NH = MODE == PF_FLAT ? f.NH : a.NH;
    const int kv_mul = MODE == PF_FLAT ? f.kv_mul : a.NH / a.NKV;
    /* scores in base 2: softmax weights by v_exp_f32 (exp2) of
     * s * scale * log2(e), one instruction instead of expf's reduction */
    const float sl2 = (MODE == PF_FLAT ? f.scale : a.scale) * 1.44269504088896341f;
    /* the last blocks of the prompt have the most keys: they take the first
     * workgroup slots, and the short ones fill in behind them */
    const int h = blockIdx.x, p0 = (int)(gridDim.y - 1 - blockIdx.y) * PQB;
    const int t = threadIdx.x, wave = t >> 6, lane = t & 63;
    const int col = lane & 15, grp = lane >> 4; /* MFMA column (query / key row) and lane group */
    const int kh = h / kv_mul;
    const int p = p0 + col; /* this lane's query position */
    if (MODE == PF_FLAT || q_roped) { /* q already rotated */
        const float* Q = MODE == PF_FLAT ? f.Q : q;
        for (int i = t; i < PQB * HD; i += PNT) {
            const int r = i / HD, e = i - r * HD;
            Qs[i] = Q[((size_t)min(p0 + r, n - 1) * NH + h) * HD + e];
        }
    } else {
        for (int i = t; i < PQB * (HD / 2); i += PNT) {
            const int r = i / (HD / 2), e = i - r * (HD / 2);
            const int pp = min(p0 + r, n - 1);
            const float ang = (float)pp * a.inv_freq[e];
            const float c = cosf(ang), sn = sinf(ang);
            const size_t qr = (size_t)pp * NH * HD + h * HD;
            const float q0 = q[qr + e];
            const float q1 = q[qr + e + HD / 2];
            Qs[r * HD + e] = q0 * c - q1 * sn;
            Qs[r * HD + e + HD / 2] = q0 * sn + q1 * c;
        }
    }
    __syncthreads();
    /* Q^T fragment: step s holds q[col][16*grp + s] */
    float qf[16];
#pragma unroll
    for (int s = 0; s < 16; s++) qf[s] = Qs[col * HD + 16 * grp + s];
    bmv_f32x4 acc[4]; /* O^T tile t: dims 16t + 4*grp + v, query col */
#pragma unroll
    for (int i = 0; i < 4; i++) acc[i] = bmv_f32x4{0.f, 0.f, 0.f, 0.f};
    float m = -INFINITY, l = 0.0f; /* m: per query (same in the 4 lane groups); l: this lane's keys */
    /* K source: dims 4g..4g+3 of key j at ksrc + j * kstr + g * kgstr (floats); V: row j at vsrc + j * vstr */
    const float *ksrc, *vsrc;
    size_t kstr, kgstr, vstr;
    if (MODE == PF_FLAT) {
        const size_t KVW = (size_t)f.NKV * HD;
        ksrc = f.K + kh * HD;
        kstr = KVW;
        kgstr = 4;
        vsrc = f.V + kh * HD;
        vstr = KVW;
    } else {
        const size_t slab = (size_t)a.MS * a.KV;
        ksrc = a.kvc + (size_t)a.layer * 2 * slab + (size_t)kh * HD * a.MS;
        kstr = 4;
        kgstr = (size_t)a.MS * 4;
        vsrc = a.kvc + ((size_t)a.layer * 2 + 1) * slab + kh * HD;
        vstr = a.KV;
    }
    /* Chunk staging: each thread moves SPT float4 of K (element i: dims
     * 4*(i / PKC), key i % PKC, so a wave reads consecutive keys of one
     * cache row) and of V (element i = 64 w + l: keys 16 (w % 4) + l % 16,
     * dims 4 (4 (w / 4) + l / 16): a wave instruction covers 16 keys x 16
     * dims, so its transposed writes into Vt fall in distinct banks; with
     * whole rows per instruction they conflicted 8 ways, 0.7 us per chunk).
     * The loads of chunk c+1 are issued into registers before chunk c is
     * computed, unconditionally (key clamped to n-1; keys at or past n
     * become zeros when written to LDS). */
    constexpr int SPT = PKC * HD4 / PNT;
    static_assert(HD4 == 16 && PKC % 16 == 0, "V staging map: 16 dim groups, 16-key runs");
    auto vkey = [](int i) { return 16 * ((i >> 6) % (PKC / 16)) + (i & 15); };
    auto vgrp = [](int i) { return 4 * ((i >> 6) / (PKC / 16)) + ((i & 63) >> 4); };
    float4 kreg[SPT], vreg[SPT];
    auto fetch = [&](int c0) {
#pragma unroll
        for (int u = 0; u < SPT; u++) {
            const int i = t + PNT * u;
            const int kk = min(c0 + i % PKC, n - 1), kg = i / PKC;
            const int vk = min(c0 + vkey(i), n - 1), vg = vgrp(i);
            __builtin_memcpy(&kreg[u], __builtin_assume_aligned(ksrc + (size_t)kk * kstr + kg * kgstr, 16), 16);
            __builtin_memcpy(&vreg[u], __builtin_assume_aligned(vsrc + (size_t)vk * vstr + 4 * vg, 16), 16);
        }
    };
    const int kend = min(p0 + PQB, n); /* keys 0 .. kend-1 */
    fetch(0);
    for (int c0 = 0; c0 < kend; c0 += PKC) {
        __syncthreads(); /* the previous chunk has been read */
#pragma unroll
        for (int u = 0; u < SPT; u++) {
            const int i = t + PNT * u;
            const int kk = i % PKC, kg = i / PKC, vk = vkey(i), vg = vgrp(i);
            const bool kin = c0 + kk < n, vin = c0 + vk < n;
            const float4 kv = kreg[u], vv = vreg[u];
            *(float4*)&Ks[kk * LDK + 4 * kg] =
                make_float4(kin ? kv.x : 0.f, kin ? kv.y : 0.f, kin ? kv.z : 0.f, kin ? kv.w : 0.f);
            Vt[(4 * vg + 0) * LDVT + vk] = vin ? vv.x : 0.f;
            Vt[(4 * vg + 1) * LDVT + vk] = vin ? vv.y : 0.f;
            Vt[(4 * vg + 2) * LDVT + vk] = vin ? vv.z : 0.f;
            Vt[(4 * vg + 3) * LDVT + vk] = vin ? vv.w : 0.f;
        }
        __syncthreads();
        if (c0 + PKC < kend) fetch(c0 + PKC);
        for (int sb = wave; sb < NSB; sb += PNW) {
            const int k0 = c0 + 16 * sb; /* first key of the sub-block */
            if (k0 >= kend) break;       /* past every query of the block (wave-uniform) */
            /* S^T[key 4*grp + v][query col] */
            /* four independent chains over the 64 dimensions (a single
             * chain of 16 dependent MFMAs waits out each one's latency) */
            bmv_f32x4 sq[4];
            const float* kr = &Ks[(16 * sb + col) * LDK + 16 * grp];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float4 k4 = *(const float4*)&kr[4 * i];
                sq[i] = __builtin_amdgcn_mfma_f32_16x16x4f32(k4.x, qf[4 * i + 0], bmv_f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
            }
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float4 k4 = *(const float4*)&kr[4 * i];
                sq[i] = __builtin_amdgcn_mfma_f32_16x16x4f32(k4.y, qf[4 * i + 1], sq[i], 0, 0, 0);
            }
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float4 k4 = *(const float4*)&kr[4 * i];
                sq[i] = __builtin_amdgcn_mfma_f32_16x16x4f32(k4.z, qf[4 * i + 2], sq[i], 0, 0, 0);
            }
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float4 k4 = *(const float4*)&kr[4 * i];
                sq[i] = __builtin_amdgcn_mfma_f32_16x16x4f32(k4.w, qf[4 * i + 3], sq[i], 0, 0, 0);
            }
            const bmv_f32x4 st = (sq[0] + sq[1]) + (sq[2] + sq[3]);
            float sv[4];
            float cm = -INFINITY;
#pragma unroll
            for (int v = 0; v < 4; v++) {
                sv[v] = k0 + 4 * grp + v <= p ? st[v] * sl2 : -INFINITY;
                cm = fmaxf(cm, sv[v]);
            }
            cm = fmaxf(cm, __shfl_xor(cm, 16));
            cm = fmaxf(cm, __shfl_xor(cm, 32));
            const float mn = fmaxf(m, cm);
            const bool live = mn > -INFINITY; /* some key of this query admitted so far */
            const float fr = live ? __builtin_amdgcn_exp2f(m - mn) : 1.0f;
            float pv[4];
#pragma unroll
            for (int v = 0; v < 4; v++) pv[v] = live ? __builtin_amdgcn_exp2f(sv[v] - mn) : 0.0f;
            l = l * fr + ((pv[0] + pv[1]) + (pv[2] + pv[3]));
#pragma unroll
            for (int ti = 0; ti < 4; ti++) acc[ti] *= fr;
            m = live ? mn : m;
            /* O^T[dim 16t + col'][query] += V^T[dim][key 4*grp + s] * P^T[key][query] */
#pragma unroll
            for (int ti = 0; ti < 4; ti++) {
                const float4 v4 = *(const float4*)&Vt[(16 * ti + col) * LDVT + 16 * sb + 4 * grp];
                acc[ti] = __builtin_amdgcn_mfma_f32_16x16x4f32(v4.x, pv[0], acc[ti], 0, 0, 0);
                acc[ti] = __builtin_amdgcn_mfma_f32_16x16x4f32(v4.y, pv[1], acc[ti], 0, 0, 0);
                acc[ti] = __builtin_amdgcn_mfma_f32_16x16x4f32(v4.z, pv[2], acc[ti], 0, 0, 0);
                acc[ti] = __builtin_amdgcn_mfma_f32_16x16x4f32(v4.w, pv[3], acc[ti], 0, 0, 0);
            }
        }
    }
    /* this wave's sum over its keys: add the four lane groups */
    l += __shfl_xor(l, 16);
    l += __shfl_xor(l, 32);
    __syncthreads(); /* every wave is done with Ks */
    float* Ws = Ks; /* [wave][dim][query] */
#pragma unroll
    for (int ti = 0; ti < 4; ti++)
#pragma unroll
        for (int v = 0; v < 4; v++) Ws[(wave * HD + 16 * ti + 4 * grp + v) * PQB + col] = acc[ti][v];
    if (grp == 0) {
        Ms[wave * PQB + col] = m;
        Ls[wave * PQB + col] = l;
    }
    __syncthreads();
    const int r = t / HD4, g = t - r * HD4; /* query r, dimensions 4g .. 4g+3 */
    if (r >= PQB || p0 + r >= n) return;
    float mx = -INFINITY;
#pragma unroll
    for (int w = 0; w < PNW; w++) mx = fmaxf(mx, Ms[w * PQB + r]);
    float den = 0.f, o0 = 0.f, o1 = 0.f, o2 = 0.f, o3 = 0.f;
#pragma unroll
    for (int w = 0; w < PNW; w++) {
        const float mv = Ms[w * PQB + r];
        const float fr = mv == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(mv - mx);
        const float* src = &Ws[(w * HD + 4 * g) * PQB + r];
        den = fmaf(fr, Ls[w * PQB + r], den);
        o0 = fmaf(fr, src[0 * PQB], o0);
        o1 = fmaf(fr, src[1 * PQB], o1);
        o2 = fmaf(fr, src[2 * PQB], o2);
        o3 = fmaf(fr, src[3 * PQB], o3);
    }
    const size_t off = ((size_t)(p0 + r) * NH + h) * HD + 4 * g;
    if (MODE == PF_FLAT) {
        f.out[off + 0] = o0 / den;
        f.out[off + 1] = o1 / den;
        f.out[off + 2] = o2 / den;
        f.out[off + 3] = o3 / den;
    } else { /* the o projection's operand: fragment order, four consecutive values */
        const uint2 o = make_uint2((unsigned int)bf16_bits(o0 / den) | ((unsigned int)bf16_bits(o1 / den) << 16),
                                   (unsigned int)bf16_bits(o2 / den) | ((unsigned int)bf16_bits(o3 / den) << 16));
        *(uint2*)(out16 + frag_index(p0 + r, h * HD + 4 * g, (NH * HD + 63) >> 6)) = o;
    }
}

__global__ __launch_bounds__(PNT) void k_pf_attn_blk(DecAttn a, const float* __restrict__ q,
                                                    unsigned short* __restrict__ out16, int n, int q_roped) {
    const PfFlat f = {};
    pf_attn_block<PF_ENGINE>(a, f, q, out16, n, q_roped);
}

__global__ __launch_bounds__(PNT) void k_attn_prefill64(PfFlat f) {
    const DecAttn a = {};
    pf_attn_block<PF_FLAT>(a, f, nullptr, nullptr, f.S, 0);
}

/* Any head size up to 128 on the reference's prefill attention ABI: one
 * wave per (query position, head); lane owns dimensions lane and lane + 64;
 * online softmax over keys 0..i with a wave-wide sum per score. */
__global__ __launch_bounds__(NT) void k_attn_prefill_wave(PfFlat f, int HD) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int i = blockIdx.y * 4 + wave, h = blockIdx.x;
    if (i >= f.S) return;
    const int kh = h / f.kv_mul;
    const size_t KVW = (size_t)f.NKV * HD;
    const float* qi = f.Q + ((size_t)i * f.NH + h) * HD;
    const bool d0 = lane < HD, d1 = lane + 64 < HD;
    const float q0 = d0 ? qi[lane] : 0.f, q1 = d1 ? qi[lane + 64] : 0.f;
    float a0 = 0.f, a1 = 0.f, m = -INFINITY, l = 0.f;
    for (int j = 0; j <= i; j++) {
        const float* kj = f.K + (size_t)j * KVW + kh * HD;
        float part = (d0 ? q0 * kj[lane] : 0.f) + (d1 ? q1 * kj[lane + 64] : 0.f);
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) part += __shfl_xor(part, o);
        const float sc = part * f.scale;
        const float mn = fmaxf(m, sc);
        const float al = expf(m - mn), be = expf(sc - mn);
        l = l * al + be;
        const float* vj = f.V + (size_t)j * KVW + kh * HD;
        if (d0) a0 = a0 * al + be * vj[lane];
        if (d1) a1 = a1 * al + be * vj[lane + 64];
        m = mn;
    }
    float* oi = f.out + ((size_t)i * f.NH + h) * HD;
    if (d0) oi[lane] = a0 / l;
    if (d1) oi[lane + 64] = a1 / l;
}

} // namespace

/* Inverse frequency of every rotary pair i < HD/2 (reference
 * src/kernels/forward.metal:1260-1279, including the llama3 frequency
 * scaling selected by r[5]), evaluated on the host in fp32 with the C
 * library's powf.  The table, not theta, goes to the device: the angle
 * (float)pos * inv is taken in fp32, so a one-ulp difference in inv moves
 * the angle by about pos ulps, and a host table keeps the frequencies
 * bit-identical to the CPU oracle's. */
extern "C" void bmk_rope_table(const float r[6], int hd, float* inv_out) {
    for (int i = 0; i < hd / 2; i++) {
        float inv = 1.0f / powf(r[0], (float)(2 * i) / (float)hd);
        if (r[5] > 0.5f) {
            const float pi = 3.14159265358979323846f;
            const float factor = r[1], low = r[2], high = r[3], orig = r[4];
            const float wavelen = 2.0f * pi / inv;
            const float low_w = orig / low, high_w = orig / high;
            if (wavelen > low_w) inv /= factor;
            if (wavelen >= high_w && wavelen <= low_w) {
                const float smooth = (orig / wavelen - low) / (high - low);
                inv = (1.0f - smooth) * inv / factor + smooth * inv;
            }
        }
        inv_out[i] = inv;
    }
}

/* ================================================================== */
/* Launchers of the reference-named kernels (buffer orders: reference
 * src/baremetal/scheduler.c:835-947). */

/* rmsnorm_forward_v2 {inp [N][C], weight [C], out [N][C], params int{N, C}, eps float} */
extern "C" int bmk_launch_rmsnorm(const bmk_launch_t* a) {
    BMK_NEED_BYTES(a, 3, 8, "params");
    BMK_NEED_BYTES(a, 4, 4, "eps");
    const int N = bmk_pi(a, 3, 0), C = bmk_pi(a, 3, 1);
    const float eps = bmk_pf(a, 4, 0);
    BMK_REQUIRE(N >= 0 && C > 0, "rmsnorm: bad shape N=%d C=%d", N, C);
    if (N == 0) return 0;
    BMK_NEED_BYTES(a, 0, (size_t)N * C * 4, "inp");
    BMK_NEED_BYTES(a, 1, (size_t)C * 4, "weight");
    BMK_NEED_BYTES(a, 2, (size_t)N * C * 4, "out");
    hipLaunchKernelGGL(k_rmsnorm, dim3(N), dim3(NT), 0, a->stream, (const float*)a->dev[0], (const float*)a->dev[1],
                       (float*)a->dev[2], C, eps);
    BMK_LAUNCH_CHECK();
    return 0;
}

/* rope_forward {q [NH][HD], k [NKV][HD], head_size int, pos int, rope float[6], n_kv_heads int};
 * NH is the Metal grid width (one thread per head, reference scheduler.c:982-984). */
extern "C" int bmk_launch_rope(const bmk_launch_t* a) {
    BMK_NEED_BYTES(a, 2, 4, "head_size");
    BMK_NEED_BYTES(a, 3, 4, "pos");
    BMK_NEED_BYTES(a, 4, 24, "rope");
    BMK_NEED_BYTES(a, 5, 4, "n_kv_heads");
    const int HD = bmk_pi(a, 2, 0), pos = bmk_pi(a, 3, 0), NKV = bmk_pi(a, 5, 0), NH = a->grid[0];
    BMK_REQUIRE(HD > 0 && HD % 2 == 0 && NH >= 0 && NKV >= 0 && NKV <= NH && pos >= 0,
                "rope: bad shape HD=%d NH=%d NKV=%d pos=%d", HD, NH, NKV, pos);
    if (NH == 0) return 0;
    BMK_NEED_BYTES(a, 0, (size_t)NH * HD * 4, "q");
    BMK_NEED_BYTES(a, 1, (size_t)NKV * HD * 4, "k");
    BMK_REQUIRE(HD <= DEC_MAX_HD, "rope: head_size %d above %d", HD, DEC_MAX_HD);
    float r[6];
    for (int i = 0; i < 6; i++) r[i] = bmk_pf(a, 4, i);
    RopeTab rt;
    bmk_rope_table(r, HD, rt.inv);
    const int n = NH * (HD / 2);
    hipLaunchKernelGGL(k_rope, dim3((n + NT - 1) / NT), dim3(NT), 0, a->stream, (float*)a->dev[0], (float*)a->dev[1],
                       NH, NKV, HD, pos, rt);
    BMK_LAUNCH_CHECK();
    return 0;
}

/* rope_forward_seq {q [S][NH][HD], k [S][NKV][HD], params int{head_size,
 * n_kv_heads, S, NH}, rope[6]} (reference forward.metal:2218-2257, the
 * prefill graph's RoPE, scheduler.c:1097-1098): q and k of every position s
 * rotated in place by angle s * inv_freq, inv_freq as rope_forward's. */
extern "C" int bmk_launch_rope_seq(const bmk_launch_t* a) {
    BMK_NEED_BYTES(a, 2, 16, "params");
    BMK_NEED_BYTES(a, 3, 24, "rope");
    const int HD = bmk_pi(a, 2, 0), NKV = bmk_pi(a, 2, 1), S = bmk_pi(a, 2, 2), NH = bmk_pi(a, 2, 3);
    BMK_REQUIRE(HD > 0 && HD % 2 == 0 && HD <= DEC_MAX_HD && NH >= 0 && NKV >= 0 && NKV <= NH && S >= 0,
                "rope_forward_seq: bad shape HD=%d NH=%d NKV=%d S=%d", HD, NH, NKV, S);
    if (NH == 0 || S == 0) return 0;
    BMK_NEED_BYTES(a, 0, (size_t)S * NH * HD * 4, "q");
    BMK_NEED_BYTES(a, 1, (size_t)S * NKV * HD * 4, "k");
    float r[6];
    for (int i = 0; i < 6; i++) r[i] = bmk_pf(a, 3, i);
    RopeTab rt;
    bmk_rope_table(r, HD, rt.inv);
    const long n = (long)S * NH * (HD / 2);
    BMK_REQUIRE(n / NT < 0x7fffffffL, "rope_forward_seq: %ld rotations", n);
    hipLaunchKernelGGL(k_rope_seq, dim3((unsigned)((n + NT - 1) / NT)), dim3(NT), 0, a->stream, (float*)a->dev[0],
                       (float*)a->dev[1], S, NH, NKV, HD, rt);
    BMK_LAUNCH_CHECK();
    return 0;
}

/* kv_store {kv cache [L][2][MS][KV], k [KV], v [KV], params int{layer, pos, MS, KV}} */
extern "C" int bmk_launch_kv_store(const bmk_launch_t* a) {
    BMK_NEED_BYTES(a, 3, 16, "params");
    const int layer = bmk_pi(a, 3, 0), pos = bmk_pi(a, 3, 1), MS = bmk_pi(a, 3, 2), KV = bmk_pi(a, 3, 3);
    BMK_REQUIRE(layer >= 0 && MS > 0 && pos >= 0 && pos < MS && KV >= 0, "kv_store: bad params layer=%d pos=%d MS=%d KV=%d",
                layer, pos, MS, KV);
    if (KV == 0) return 0;
    BMK_NEED_BYTES(a, 0, ((size_t)layer * 2 + 2) * MS * KV * 4, "kv cache");
    BMK_NEED_BYTES(a, 1, (size_t)KV * 4, "k");
    BMK_NEED_BYTES(a, 2, (size_t)KV * 4, "v");
    hipLaunchKernelGGL(k_kv_store, dim3((KV + NT - 1) / NT), dim3(NT), 0, a->stream, (float*)a->dev[0],
                       (const float*)a->dev[1], (const float*)a->dev[2], layer, pos, MS, KV);
    BMK_LAUNCH_CHECK();
    return 0;
}

/* attention_forward {q [NH][HD], kv cache, out [NH][HD],
 *                    params int{NH, HD, NKV, KV, S, kv_mul, layer, MS}, scale float} */
extern "C" int bmk_launch_attention(const bmk_launch_t* a) {
    BMK_NEED_BYTES(a, 3, 32, "params");
    BMK_NEED_BYTES(a, 4, 4, "scale");
    const int NH = bmk_pi(a, 3, 0), HD = bmk_pi(a, 3, 1), KV = bmk_pi(a, 3, 3), S = bmk_pi(a, 3, 4);
    const int kv_mul = bmk_pi(a, 3, 5), layer = bmk_pi(a, 3, 6), MS = bmk_pi(a, 3, 7);
    const float scale = bmk_pf(a, 4, 0);
    BMK_REQUIRE(NH > 0 && HD > 0 && HD <= 256 && 256 % HD == 0 && HD % 4 == 0 && kv_mul > 0 && layer >= 0 && MS > 0 &&
                    S >= 1 && S <= MS && ((NH - 1) / kv_mul + 1) * HD <= KV,
                "attention: bad params NH=%d HD=%d KV=%d S=%d kv_mul=%d layer=%d MS=%d", NH, HD, KV, S, kv_mul, layer,
                MS);
    BMK_NEED_BYTES(a, 0, (size_t)NH * HD * 4, "q");
    BMK_NEED_BYTES(a, 1, ((size_t)layer * 2 + 2) * MS * KV * 4, "kv cache");
    BMK_NEED_BYTES(a, 2, (size_t)NH * HD * 4, "out");
    BMK_REQUIRE(((uintptr_t)a->dev[1] & 15) == 0 && KV % 4 == 0, "attention: kv cache rows must be 16-byte aligned");
    hipLaunchKernelGGL(k_attention, dim3(NH), dim3(NT), 0, a->stream, (const float*)a->dev[0], (const float*)a->dev[1],
                       (float*)a->dev[2], HD, KV, S, kv_mul, layer, MS, scale);
    BMK_LAUNCH_CHECK();
    return 0;
}

/* attention_forward_prefill / _warp / _tiled (reference forward.metal:1904-2114,
 * selected by scheduler.c:1081-1089 in prefill mode):
 * {Q [S][NH][HD] (roped), K [S][NKV][HD], V [S][NKV][HD], out [S][NH][HD],
 *  params int{NH, S, HD, NKV, kv_mul}, scale}.  Causal softmax(Q K^T * scale) V
 * per head, head h reading KV head h / kv_mul.  Head size 64: blocks of 16
 * positions per workgroup; other head sizes up to 128: one wave per
 * (position, head).  The reference's kernels return without writing on a
 * head size they do not handle; here such a request is an error. */
extern "C" int bmk_launch_attention_prefill(const bmk_launch_t* a) {
    BMK_NEED_BYTES(a, 4, 20, "params");
    BMK_NEED_BYTES(a, 5, 4, "scale");
    PfFlat f;
    f.NH = bmk_pi(a, 4, 0);
    f.S = bmk_pi(a, 4, 1);
    const int HD = bmk_pi(a, 4, 2);
    f.NKV = bmk_pi(a, 4, 3);
    f.kv_mul = bmk_pi(a, 4, 4);
    f.scale = bmk_pf(a, 5, 0);
    BMK_REQUIRE(f.NH > 0 && f.S >= 0 && HD > 0 && HD <= 128 && f.NKV > 0 && f.kv_mul > 0 &&
                    (f.NH - 1) / f.kv_mul < f.NKV,
                "attention prefill: bad params NH=%d S=%d HD=%d NKV=%d kv_mul=%d", f.NH, f.S, HD, f.NKV, f.kv_mul);
    if (f.S == 0) return 0;
    const size_t qn = (size_t)f.S * f.NH * HD, kn = (size_t)f.S * f.NKV * HD;
    BMK_NEED_BYTES(a, 0, qn * 4, "Q");
    BMK_NEED_BYTES(a, 1, kn * 4, "K");
    BMK_NEED_BYTES(a, 2, kn * 4, "V");
    BMK_NEED_BYTES(a, 3, qn * 4, "out");
    f.Q = (const float*)a->dev[0];
    f.K = (const float*)a->dev[1];
    f.V = (const float*)a->dev[2];
    f.out = (float*)a->dev[3];
    const bool aligned = (((uintptr_t)a->dev[0] | (uintptr_t)a->dev[1] | (uintptr_t)a->dev[2] | (uintptr_t)a->dev[3]) & 15) == 0;
    if (HD == 64 && aligned)
        hipLaunchKernelGGL(k_attn_prefill64, dim3(f.NH, (f.S + PQB - 1) / PQB), dim3(PNT), 0, a->stream, f);
    else
        hipLaunchKernelGGL(k_attn_prefill_wave, dim3(f.NH, (f.S + 3) / 4), dim3(NT), 0, a->stream, f, HD);
    BMK_LAUNCH_CHECK();
    return 0;
}

/* add_forward {a, b, out, n int} */
extern "C" int bmk_launch_add(const bmk_launch_t* a) {
    BMK_NEED_BYTES(a, 3, 4, "n");
    const int n = bmk_pi(a, 3, 0);
    BMK_REQUIRE(n >= 0, "add: n=%d", n);
    if (n == 0) return 0;
    for (int i = 0; i < 3; i++) BMK_NEED_BYTES(a, i, (size_t)n * 4, "operand");
    hipLaunchKernelGGL(k_add, dim3((n + NT - 1) / NT), dim3(NT), 0, a->stream, (const float*)a->dev[0],
                       (const float*)a->dev[1], (float*)a->dev[2], n);
    BMK_LAUNCH_CHECK();
    return 0;
}

/* swiglu_forward {gate, up, out, N int} */
extern "C" int bmk_launch_swiglu(const bmk_launch_t* a) {
    BMK_NEED_BYTES(a, 3, 4, "N");
    const int n = bmk_pi(a, 3, 0);
    BMK_REQUIRE(n >= 0, "swiglu: N=%d", n);
    if (n == 0) return 0;
    for (int i = 0; i < 3; i++) BMK_NEED_BYTES(a, i, (size_t)n * 4, "operand");
    hipLaunchKernelGGL(k_swiglu, dim3((n + NT - 1) / NT), dim3(NT), 0, a->stream, (const float*)a->dev[0],
                       (const float*)a->dev[1], (float*)a->dev[2], n);
    BMK_LAUNCH_CHECK();
    return 0;
}

static int head_tiles(int D, int V, int wf) {
    const int nseg = wf == HW_F32 ? D / 16 : D / 32;
    const int rows = (NT / nseg) * head_u(wf);
    return (V + rows - 1) / rows;
}

static bool head_shape_ok(int D, int wf) {
    return wf == HW_F32 ? (D % 16 == 0 && D / 16 <= NT) : (D % 32 == 0 && D / 32 <= NT);
}

/* rmsnorm_matmul_forward (fp32 wcls) and rmsnorm_matmul_forward_bf16_vec
 * (bf16 wcls): {x [C], norm weight [C], wcls [V][C], logits [V],
 * params int{C, V}, eps float} (reference forward.metal:1532-1581,
 * 1636-1689; scheduler.c:931-940).  The grid the caller passes is not used:
 * the launch covers V rows by itself. */
/* k_head over one of the unquantized row formats */
static void launch_head_rows(const DecHead& h, int wf, hipStream_t s) {
    if (wf == HW_F32) hipLaunchKernelGGL(k_head<HW_F32>, dim3(h.tiles), dim3(NT), 0, s, h);
    else if (wf == HW_BF16) hipLaunchKernelGGL(k_head<HW_BF16>, dim3(h.tiles), dim3(NT), 0, s, h);
    else hipLaunchKernelGGL(k_head<HW_F16>, dim3(h.tiles), dim3(NT), 0, s, h);
}

static const char* row_format_name(int wf) { return wf == HW_F32 ? "fp32" : wf == HW_BF16 ? "bf16" : "fp16"; }

/* RMSNorm + matmul for any C the LM-head kernel does not tile: one
 * workgroup per output row, the RMS of x recomputed in each (x is short
 * next to a row of the head), the dot product strided over C. */
template <int WF>
__global__ __launch_bounds__(NT) void k_rmsnorm_matmul_rows_any(const float* __restrict__ x,
                                                                const float* __restrict__ g, const void* __restrict__ w,
                                                                float* __restrict__ out, int C, float eps) {
    __shared__ float sh[NT / 64];
    const int r = blockIdx.x;
    float ss = 0.f;
    for (int k = threadIdx.x; k < C; k += NT) ss = fmaf(x[k], x[k], ss);
    const float inv = 1.0f / sqrtf(block_sum(ss, sh) / (float)C + eps);
    const float* wf = (const float*)w + (size_t)r * C;
    const unsigned short* wh = (const unsigned short*)w + (size_t)r * C;
    float s = 0.f;
    for (int k = threadIdx.x; k < C; k += NT) {
        const float wv = WF == HW_F32 ? wf[k] : h16_lo<WF>(wh[k]);
        s = fmaf((x[k] * inv) * g[k], wv, s);
    }
    s = block_sum(s, sh);
    if (threadIdx.x == 0) out[r] = s;
}

/* rmsnorm_matmul_forward{,_bf16,_bf16_vec,_fp16,_fp16_vec} {x [C], norm
 * weight [C], wcls [V][C] (fp32, bf16 or fp16), logits [V], params
 * int{C, V}, eps} (reference forward.metal:1532-1581, 1585-1634,
 * 1636-1689, 1692-1745, 1748-1801): the fused final norm and LM head.  The LM-head kernel where
 * it tiles C (fp32 rows: a multiple of 16 up to 4096; 16-bit rows: of 32 up
 * to 8192), k_rmsnorm_matmul_rows_any for any other C. */
static int launch_rmsnorm_matmul(const bmk_launch_t* a, int wf) {
    const char* name = wf == HW_F32 ? "rmsnorm_matmul" : wf == HW_BF16 ? "rmsnorm_matmul_bf16" : "rmsnorm_matmul_fp16";
    const size_t esz = wf == HW_F32 ? 4 : 2;
    BMK_NEED_BYTES(a, 4, 8, "params");
    BMK_NEED_BYTES(a, 5, 4, "eps");
    const int C = bmk_pi(a, 4, 0), V = bmk_pi(a, 4, 1);
    BMK_REQUIRE(C > 0 && V >= 0, "%s: C=%d V=%d", name, C, V);
    if (V == 0) return 0;
    BMK_NEED_BYTES(a, 0, (size_t)C * 4, "x");
    BMK_NEED_BYTES(a, 1, (size_t)C * 4, "norm weight");
    BMK_NEED_BYTES(a, 2, (size_t)V * C * esz, "wcls");
    BMK_NEED_BYTES(a, 3, (size_t)V * 4, "logits");
    if (!head_shape_ok(C, wf)) {
        BMK_REQUIRE((((uintptr_t)a->dev[0] | (uintptr_t)a->dev[1]) & 3) == 0 && ((uintptr_t)a->dev[2] & (esz - 1)) == 0,
                    "%s: misaligned operand", name);
        const float* x = (const float*)a->dev[0];
        const float* g = (const float*)a->dev[1];
        float* out = (float*)a->dev[3];
        const float eps = bmk_pf(a, 5, 0);
        if (wf == HW_F32)
            hipLaunchKernelGGL(k_rmsnorm_matmul_rows_any<HW_F32>, dim3(V), dim3(NT), 0, a->stream, x, g,
                               (const void*)a->dev[2], out, C, eps);
        else if (wf == HW_BF16)
            hipLaunchKernelGGL(k_rmsnorm_matmul_rows_any<HW_BF16>, dim3(V), dim3(NT), 0, a->stream, x, g,
                               (const void*)a->dev[2], out, C, eps);
        else
            hipLaunchKernelGGL(k_rmsnorm_matmul_rows_any<HW_F16>, dim3(V), dim3(NT), 0, a->stream, x, g,
                               (const void*)a->dev[2], out, C, eps);
        BMK_LAUNCH_CHECK();
        return 0;
    }
    BMK_REQUIRE((((uintptr_t)a->dev[0] | (uintptr_t)a->dev[1] | (uintptr_t)a->dev[2]) & 3) == 0,
                "%s: misaligned operand", name);
    DecHead h;
    memset(&h, 0, sizeof h);
    h.x = (const float*)a->dev[0];
    h.norm_w = (const float*)a->dev[1];
    if (wf == HW_F32) h.w = (const float*)a->dev[2];
    else h.wh = (const unsigned short*)a->dev[2];
    h.logits = (float*)a->dev[3];
    h.D = C;
    h.V = V;
    h.B = 1;
    h.eps = bmk_pf(a, 5, 0);
    h.tiles = head_tiles(C, V, wf);
    launch_head_rows(h, wf, a->stream);
    BMK_LAUNCH_CHECK();
    return 0;
}

extern "C" int bmk_launch_rmsnorm_matmul(const bmk_launch_t* a) { return launch_rmsnorm_matmul(a, HW_F32); }
extern "C" int bmk_launch_rmsnorm_matmul_bf16(const bmk_launch_t* a) { return launch_rmsnorm_matmul(a, HW_BF16); }
extern "C" int bmk_launch_rmsnorm_matmul_fp16(const bmk_launch_t* a) { return launch_rmsnorm_matmul(a, HW_F16); }

/* The plain matmul for any C the LM-head kernel does not tile: one
 * workgroup per output row r, the BT input rows in turn, each dot product
 * strided over C by the 256 threads with fp32 sums (as the reference's
 * naive kernel, forward.metal:23-37, one thread per output). */
template <int WF>
__global__ __launch_bounds__(NT) void k_matmul_rows_any(const float* __restrict__ x, const void* __restrict__ w,
                                                        const float* __restrict__ bias, float* __restrict__ out,
                                                        int BT, int C, int OC) {
    __shared__ float sh[NT / 64];
    const int r = blockIdx.x;
    const float* wf = (const float*)w + (size_t)r * C;
    const unsigned short* wh = (const unsigned short*)w + (size_t)r * C;
    for (int b = 0; b < BT; b++) {
        const float* xb = x + (size_t)b * C;
        float s = 0.f;
        for (int k = threadIdx.x; k < C; k += NT) {
            const float wv = WF == HW_F32 ? wf[k] : h16_lo<WF>(wh[k]);
            s = fmaf(xb[k], wv, s);
        }
        s = block_sum(s, sh);
        if (threadIdx.x == 0) out[(size_t)b * OC + r] = bias ? bias[r] + s : s;
    }
}

/* The plain fp32, bf16 and fp16 matmul kernels: {inp [BT][C], weight
 * [OC][C] (fp32, bf16 or fp16), bias [OC], out [BT][OC], params int{BT, C,
 * OC, has_bias}} (reference forward.metal:23-37 matmul_forward_naive,
 * 513-560 matmul_forward_tiled, 449-503 matmul_forward_fp32_tiled, 52-89
 * matmul_forward_bf16_vec, 91-110 matmul_forward_bf16, 116-319
 * matmul_forward_bf16_tiled / _tiled64 / _simd, 327-442
 * matmul_forward_fp16_vec / _fp16 / _fp16_tiled).  The reference's
 * prefill takes them for the LM head of its last position (graph.c:373-380,
 * selected by scheduler.c:1118-1145 and registry.c:60-67).  Served by the
 * LM-head kernel with the RMSNorm off where it tiles C (a multiple of 16 up
 * to 4096 for fp32 rows, of 32 up to 8192 for bf16): each workgroup loads
 * its weight rows once and applies them to all BT input rows.  Any other C
 * takes k_matmul_rows_any.  The grid the caller passes is not used. */
static int launch_matmul_rows(const bmk_launch_t* a, int wf) {
    const char* name = wf == HW_F32 ? "matmul_forward (fp32)" : wf == HW_BF16 ? "matmul_forward_bf16" : "matmul_forward_fp16";
    const size_t esz = wf == HW_F32 ? 4 : 2;
    BMK_NEED_BYTES(a, 4, 16, "params");
    const int BT = bmk_pi(a, 4, 0), C = bmk_pi(a, 4, 1), OC = bmk_pi(a, 4, 2), hb = bmk_pi(a, 4, 3);
    BMK_REQUIRE(BT >= 0 && OC >= 0 && C > 0, "%s: BT=%d C=%d OC=%d", name, BT, C, OC);
    if (BT == 0 || OC == 0) return 0;
    BMK_NEED_BYTES(a, 0, (size_t)BT * C * 4, "inp");
    BMK_NEED_BYTES(a, 1, (size_t)OC * C * esz, "weight");
    if (hb) BMK_NEED_BYTES(a, 2, (size_t)OC * 4, "bias");
    BMK_NEED_BYTES(a, 3, (size_t)BT * OC * 4, "out");
    if (!head_shape_ok(C, wf)) {
        BMK_REQUIRE(((uintptr_t)a->dev[0] & 3) == 0 && ((uintptr_t)a->dev[1] & (esz - 1)) == 0,
                    "%s: misaligned operand", name);
        const float* bias = hb ? (const float*)a->dev[2] : nullptr;
        if (wf == HW_F32)
            hipLaunchKernelGGL(k_matmul_rows_any<HW_F32>, dim3(OC), dim3(NT), 0, a->stream, (const float*)a->dev[0],
                               (const void*)a->dev[1], bias, (float*)a->dev[3], BT, C, OC);
        else if (wf == HW_BF16)
            hipLaunchKernelGGL(k_matmul_rows_any<HW_BF16>, dim3(OC), dim3(NT), 0, a->stream, (const float*)a->dev[0],
                               (const void*)a->dev[1], bias, (float*)a->dev[3], BT, C, OC);
        else
            hipLaunchKernelGGL(k_matmul_rows_any<HW_F16>, dim3(OC), dim3(NT), 0, a->stream, (const float*)a->dev[0],
                               (const void*)a->dev[1], bias, (float*)a->dev[3], BT, C, OC);
        BMK_LAUNCH_CHECK();
        return 0;
    }
    BMK_REQUIRE((((uintptr_t)a->dev[0] | (uintptr_t)a->dev[1]) & 3) == 0, "%s: misaligned operand", name);
    DecHead h;
    memset(&h, 0, sizeof h);
    h.x = (const float*)a->dev[0];
    if (wf == HW_F32) h.w = (const float*)a->dev[1];
    else h.wh = (const unsigned short*)a->dev[1];
    h.bias = hb ? (const float*)a->dev[2] : nullptr;
    h.logits = (float*)a->dev[3];
    h.D = C;
    h.V = OC;
    h.B = BT;
    h.tiles = head_tiles(C, OC, wf);
    launch_head_rows(h, wf, a->stream);
    BMK_LAUNCH_CHECK();
    return 0;
}

extern "C" int bmk_launch_matmul_f32(const bmk_launch_t* a) { return launch_matmul_rows(a, HW_F32); }
extern "C" int bmk_launch_matmul_bf16(const bmk_launch_t* a) { return launch_matmul_rows(a, HW_BF16); }
extern "C" int bmk_launch_matmul_fp16(const bmk_launch_t* a) { return launch_matmul_rows(a, HW_F16); }

/* argmax_f32 {values f32 [n], out int [1], params int{n}} */
extern "C" int bmk_launch_argmax(const bmk_launch_t* a) {
    BMK_NEED_BYTES(a, 2, 4, "params");
    const int n = bmk_pi(a, 2, 0);
    BMK_REQUIRE(n > 0, "argmax: n=%d", n);
    BMK_NEED_BYTES(a, 0, (size_t)n * 4, "values");
    BMK_NEED_BYTES(a, 1, 4, "out");
    hipLaunchKernelGGL(k_argmax, dim3(1), dim3(1024), 0, a->stream, (const float*)a->dev[0], n, (int*)a->dev[1]);
    BMK_LAUNCH_CHECK();
    return 0;
}

/* ================================================================== */
/* Engine-side launchers (arguments already validated by engine.cpp). */

/* Launch shape of a fused matvec phase over C columns: the smallest
 * workgroup that holds a row's C/32 block columns, one row pass per lane;
 * a SwiGLU phase keeps whole (gate, up) row pairs in a tile. */
static void dec_mv_shape(int C, int glu, int* wt, int* slots, int* u) {
    const int nb = C / 32;
    *wt = nb <= 64 ? 64 : (nb <= 128 ? 128 : 256);
    *u = 1;
    if (glu && nb <= 64) { /* gate/up of a narrow row: 128 lanes, two passes (measured fastest) */
        *wt = 128;
        *u = 2;
    }
    *slots = *wt / nb;
    if (glu && *slots == 1 && *wt < 256) { /* a pair needs two row slots */
        *wt *= 2;
        *slots = *wt / nb;
    }
    if (glu && (*slots & 1)) *slots = *slots > 1 ? *slots - 1 : 0;
}

extern "C" int dec_mv_tiles(int OC, int C, int glu) {
    int wt, slots, u;
    dec_mv_shape(C, glu, &wt, &slots, &u);
    if (slots == 0) return -1; /* a gate/up pair wider than one workgroup: not supported */
    const long n = glu ? 2L * OC : (long)OC;
    return (int)((n + (long)slots * u - 1) / ((long)slots * u));
}

/* wf: 0 fp32 rows, 1 Q8 rows, 2 bf16 rows */
extern "C" int dec_head_tiles(int D, int V, int wf) { return head_tiles(D, V, wf); }

extern "C" int dec_launch_embed(const DecEmbed* a, hipStream_t s) {
    if (a->B < 1 || a->B > DEC_MAX_B) return -1;
    hipLaunchKernelGGL(k_embed, dim3(a->B), dim3(NT), 0, s, *a); /* workgroup b: sequence b */
    BMK_LAUNCH_CHECK();
    return 0;
}

/* Workgroups of one matrix in the batched (B >= 2) matvec: 16 output rows,
 * or 8 (gate, up) row pairs. */
static int dec_bmv_tiles(int OC, int glu) { return glu ? (OC + 7) / 8 : (OC + 15) / 16; }

extern "C" int dec_launch_mv(const DecMv* a_in, hipStream_t s) {
    DecMv a = *a_in;
    if (a.B >= 2) {
        if (a.B > DEC_MAX_B || a.C % 32 || (a.ldx & 3) || ((uintptr_t)a.x & 15)) return -1;
        a.tile0[0] = 0;
        for (int i = 0; i < a.nmat; i++) a.tile0[i + 1] = a.tile0[i] + dec_bmv_tiles(a.OC[i], a.glu);
        /* one workgroup per (row tile, 16 batch rows): more workgroups than
         * one per row tile, each weight tile is read from L2 again */
        const dim3 grid(a.tile0[a.nmat], (a.B + 15) / 16);
        if (a.qf == QF_Q4) hipLaunchKernelGGL(k_dec_bmv4<1>, grid, dim3(DBMV_NT), 0, s, a);
        else hipLaunchKernelGGL(k_dec_bmv<1>, grid, dim3(DBMV_NT), 0, s, a);
        BMK_LAUNCH_CHECK();
        return 0;
    }
    int wt, u;
    dec_mv_shape(a.C, a.glu, &wt, &a.slots, &u);
    if (a.slots == 0) return -1;
    const dim3 grid(a.tile0[a.nmat]);
#define DEC_MV(K)                                                                    \
    do {                                                                             \
        if (wt == 64) hipLaunchKernelGGL((K<64, 1>), grid, dim3(64), 0, s, a);       \
        else if (wt == 128 && u == 2) hipLaunchKernelGGL((K<128, 2>), grid, dim3(128), 0, s, a); \
        else if (wt == 128) hipLaunchKernelGGL((K<128, 1>), grid, dim3(128), 0, s, a); \
        else hipLaunchKernelGGL((K<256, 1>), grid, dim3(256), 0, s, a);             \
    } while (0)
    if (a.qf == QF_Q4) DEC_MV(k_dec_mv4);
    else DEC_MV(k_dec_mv);
#undef DEC_MV
    BMK_LAUNCH_CHECK();
    return 0;
}

extern "C" int dec_launch_attn(const DecAttn* a, int B, hipStream_t s) {
    const int kvm = a->NH / a->NKV;
    /* B >= 2: one workgroup per KV-head group (K and V rows read once for the
     * group's query heads).  B = 1: one workgroup per query head, which puts
     * three times as many CUs on the step's few rows and measured faster. */
    if (B >= 2 && (a->HD == 16 || a->HD == 32 || a->HD == 64) && kvm >= 1 && kvm <= 4) {
        const dim3 g(a->NKV, B), tb(64 * AG_WAVES);
#define AG_LAUNCH(HDV)                                                                          \
        do {                                                                                    \
            if (kvm == 1) hipLaunchKernelGGL((k_dec_attn_g<HDV, 1>), g, tb, 0, s, *a);          \
            else if (kvm == 2) hipLaunchKernelGGL((k_dec_attn_g<HDV, 2>), g, tb, 0, s, *a);     \
            else if (kvm == 3) hipLaunchKernelGGL((k_dec_attn_g<HDV, 3>), g, tb, 0, s, *a);     \
            else hipLaunchKernelGGL((k_dec_attn_g<HDV, 4>), g, tb, 0, s, *a);                   \
        } while (0)
        if (a->HD == 64) AG_LAUNCH(64);
        else if (a->HD == 32) AG_LAUNCH(32);
        else AG_LAUNCH(16);
#undef AG_LAUNCH
        BMK_LAUNCH_CHECK();
        return 0;
    }
    if (a->HD == 64) hipLaunchKernelGGL(k_dec_attn1<64>, dim3(a->NH, B), dim3(NT), 0, s, *a);
    else if (a->HD == 128) hipLaunchKernelGGL(k_dec_attn<128>, dim3(a->NH, B), dim3(NT), 0, s, *a);
    else hipLaunchKernelGGL(k_dec_attn<0>, dim3(a->NH, B), dim3(NT), 0, s, *a);
    BMK_LAUNCH_CHECK();
    return 0;
}

/* LDS for the batch rows of a batched head launch at most (two workgroups per CU) */
#define HEAD_XL_BYTES (76u << 10)

extern "C" int dec_launch_head(const DecHead* a_in, hipStream_t s) {
    if (a_in->B >= 2) {
        DecHead a = *a_in;
        if (a.B > DEC_MAX_B || a.D % 32) return -1;
        a.tiles = (a.V + 63) / 64;
        const dim3 grid(a.tiles);
        const int wf = a.wq ? HW_Q8 : (a.wh ? (a.wh_f16 ? HW_F16 : HW_BF16) : HW_F32);
        /* the batch rows in LDS when they fit beside a second workgroup's */
#define HEAD_B2(NBT, XL, LDSB)                                                                             \
        do {                                                                                               \
            if (wf == HW_Q8) hipLaunchKernelGGL((k_head_b<NBT, HW_Q8, XL>), grid, dim3(NT), LDSB, s, a);        \
            else if (wf == HW_BF16) hipLaunchKernelGGL((k_head_b<NBT, HW_BF16, XL>), grid, dim3(NT), LDSB, s, a); \
            else if (wf == HW_F16) hipLaunchKernelGGL((k_head_b<NBT, HW_F16, XL>), grid, dim3(NT), LDSB, s, a);  \
            else hipLaunchKernelGGL((k_head_b<NBT, HW_F32, XL>), grid, dim3(NT), LDSB, s, a);                    \
        } while (0)
#define HEAD_B(NBT)                                                                                        \
        do {                                                                                               \
            const unsigned xb = (unsigned)a.D * NBT * 64u;                                                 \
            if (xb <= HEAD_XL_BYTES) HEAD_B2(NBT, true, xb);                                               \
            else HEAD_B2(NBT, false, 0);                                                                   \
        } while (0)
        if (a.B <= 16) HEAD_B(1);
        else if (a.B <= 32) HEAD_B(2);
        else if (a.B <= 48) HEAD_B(3);
        else HEAD_B(4);
#undef HEAD_B
#undef HEAD_B2
        BMK_LAUNCH_CHECK();
        return 0;
    }
    const DecHead* a = a_in;
    if (a->wq)
        hipLaunchKernelGGL(k_head<HW_Q8>, dim3(a->tiles), dim3(NT), 0, s, *a);
    else if (a->wh && a->wh_f16)
        hipLaunchKernelGGL(k_head<HW_F16>, dim3(a->tiles), dim3(NT), 0, s, *a);
    else if (a->wh)
        hipLaunchKernelGGL(k_head<HW_BF16>, dim3(a->tiles), dim3(NT), 0, s, *a);
    else
        hipLaunchKernelGGL(k_head<HW_F32>, dim3(a->tiles), dim3(NT), 0, s, *a);
    BMK_LAUNCH_CHECK();
    return 0;
}

/* fp32 -> IEEE fp16 over n elements, rounded to nearest even (v_cvt_f16_f32;
 * values past the fp16 range become infinities), as the reference's fp16
 * upload converts (scheduler.c:410-417) */
__global__ __launch_bounds__(NT) void k_cast_f16(const float* __restrict__ src, unsigned short* __restrict__ dst,
                                                 long n) {
    for (long i = (long)blockIdx.x * NT + threadIdx.x; i < n; i += (long)gridDim.x * NT)
        dst[i] = __builtin_bit_cast(unsigned short, (_Float16)src[i]);
}

extern "C" int dec_cast_f16(const float* src, unsigned short* dst, long n, hipStream_t s) {
    if (n <= 0) return 0;
    const long blocks = std::min<long>((n + NT - 1) / NT, 4096);
    hipLaunchKernelGGL(k_cast_f16, dim3((unsigned)blocks), dim3(NT), 0, s, src, dst, n);
    BMK_LAUNCH_CHECK();
    return 0;
}

/* ------------------------------------------------------------------ */
/* Prefill launchers (arguments validated by engine.cpp). */

extern "C" int dec_pf_embed(const int* tok, const float* emb, float* x, int n, int D, const float* g,
                            unsigned short* an, float* ss, int ss_tiles, int ss_ld, const DecAttn* ra, float* rope,
                            hipStream_t s) {
    BMK_REQUIRE(D % 32 == 0 && ss_tiles >= 1 && ss_tiles <= NT && ss_ld >= n && ((uintptr_t)an & 15) == 0,
                "prefill embedding: D %d, %d sum slots", D, ss_tiles);
    hipLaunchKernelGGL(k_pf_embed, dim3(n), dim3(NT), 0, s, tok, emb, x, D, g, an, ss, ss_tiles, ss_ld, *ra, rope);
    BMK_LAUNCH_CHECK();
    return 0;
}

/* RoPE + cache append of every position (unless the q/k/v GEMM's epilogue
 * did it, q's RoPE too: kv_done), then causal attention; the result goes to
 * out16 as bf16 in fragment order (the o-projection's operand).  Head size
 * 64: blocks of PQB positions per workgroup, written as bf16 directly; other
 * head sizes: one workgroup per (head, position) into a->out (fp32), then
 * the fragment-order cast (which also zeroes the columns past NH * HD). */
extern "C" int dec_pf_attention(const DecAttn* a, const float* q, const float* k, const float* v, int n,
                                unsigned short* out16, int kv_done, hipStream_t s) {
    if (!kv_done) {
        hipLaunchKernelGGL(k_pf_kv, dim3(n), dim3(NT), 0, s, *a, k, v);
        BMK_LAUNCH_CHECK();
    }
    if (a->HD == 64) {
        hipLaunchKernelGGL(k_pf_attn_blk, dim3(a->NH, (n + PQB - 1) / PQB), dim3(PNT), 0, s, *a, q, out16, n,
                           kv_done);
        BMK_LAUNCH_CHECK();
        return 0;
    }
    const dim3 g(a->NH, n);
    if (a->HD == 128) hipLaunchKernelGGL(k_pf_attn<128>, g, dim3(NT), 0, s, *a, q, k, v);
    else hipLaunchKernelGGL(k_pf_attn<0>, g, dim3(NT), 0, s, *a, q, k, v);
    BMK_LAUNCH_CHECK();
    return gm_cast_bf16_frag(a->out, out16, n, a->NH * a->HD, a->NH * a->HD, s);
}

