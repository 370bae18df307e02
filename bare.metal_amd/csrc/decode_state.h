/* SPDX-License-Identifier: MPL-2.0
 *
 * decode_state.h — the device-resident state of a decode session and the
 * argument blocks of the fused decode kernels (decode.hip), shared with the
 * host engine (engine.cpp).
 *
 * Every value that changes from one token to the next (position, input
 * token, argmax) lives in DecState in device memory, so the kernels of one
 * step take identical arguments at every step and the step is captured once
 * into a hipGraph and replayed.  All B sequences of a batched session are
 * at the same position (they are stepped in lockstep).
 */
#ifndef BMK_DECODE_STATE_H
#define BMK_DECODE_STATE_H

#include <hip/hip_runtime.h>

#ifdef __cplusplus
extern "C" {
#endif
/* RoPE inverse frequencies of pairs 0..hd/2-1 from r = {theta, factor,
 * low, high, original max, llama3 flag} (decode.hip). */
void bmk_rope_table(const float r[6], int hd, float* inv_out);
#ifdef __cplusplus
}
#endif

#define DEC_MAX_B 64
#define DEC_MAX_MATS 3
#define DEC_MAX_HD 256

typedef struct {
    int pos;          /* position of the step being run; the last head workgroup advances it */
    int n_prompt;     /* generation mode: prompt length */
    int n_out;        /* generation mode: steps whose argmax has been emitted */
    int host_mode;    /* 1: the input tokens come from host_token[], 0: prompt, then last_token */
    unsigned int done;/* head workgroups finished in the current step */
    int B;
    int bad_token;    /* set when an input token was outside [0, V) (0 was used instead) */
    int sync_error;   /* set (and kept) when the persistent step kernel timed out waiting for a value */
    int pad_[2];
    int token[DEC_MAX_B];        /* input token of the current step */
    int host_token[DEC_MAX_B];
    int last_token[DEC_MAX_B];   /* argmax of the last finished step */
    unsigned long long key[DEC_MAX_B]; /* running argmax of the current step, packed (value, ~index) */
} DecState;

/* One fused quantized matvec phase: y_i = W_i * f(x) for up to three matrices that
 * share the input, f = identity or RMSNorm(x) * norm_w.
 *  glu      : W_0 = gate, W_1 = up; y_0 = silu(gate x) * (up x)
 *  residual : y_0 += previous y_0 (y_0 is the residual stream, updated in place)
 * Batched: B input rows (stride ldx); y_i row b at y_i + b * OC_i. */
typedef struct {
    const float* x;
    const float* norm_w;       /* NULL: no norm */
    float eps;
    int C;
    int B;
    int ldx;
    int nmat;
    int glu;
    int residual;
    int slots;                 /* rows per row pass of a workgroup (set by the launcher; even for glu) */
    int qf;                    /* weight blocks: 0 Q8_0 (36 bytes), 1 Q4_0 (20 bytes) */
    const unsigned char* w[DEC_MAX_MATS];
    float* y[DEC_MAX_MATS];
    int OC[DEC_MAX_MATS];
    int tile0[DEC_MAX_MATS + 1];   /* workgroup prefix: matrix i owns tiles tile0[i] .. tile0[i+1]-1 */
} DecMv;

/* Rope + KV append + GQA attention for one layer of a decode step.  The
 * cache is [B][L][2][MS*KV]: per (sequence, layer) first K, per KV head
 * [HD/4][MS] float4 (4 dimensions of one position per 16 bytes), then V
 * row-major ([MS][KV]). */
typedef struct {
    const float* q;     /* [B][NH*HD] un-roped */
    const float* k;     /* [B][KV] un-roped */
    const float* v;     /* [B][KV] */
    float* kvc;
    float* out;         /* [B][NH*HD] */
    const DecState* st;
    float inv_freq[DEC_MAX_HD / 2]; /* RoPE inverse frequency per rotary pair (host table) */
    float scale;
    int NH, NKV, HD, KV, MS, L, layer;
} DecAttn;

/* Where the workgroups of an LM head launch meet: HEAD_GROUPS groups
 * (workgroup w in group w % HEAD_GROUPS), each with its arrival counter on
 * a 256-byte line of its own and its running argmax keys; the last arrival
 * of a group folds the group's keys into DecState.key and counts the group
 * at [HEAD_GROUPS].  Same-address device-scope atomics queue up where the
 * XCDs meet (about 10 ns apart): one counter for all of a launch's 768
 * workgroups cost 8 us, sixteen on separate lines under 1 us.  Zeroed when
 * allocated; every counter and key is re-armed by the arrival that reads
 * it. */
#define HEAD_GROUPS 16
typedef struct {
    unsigned int cnt[HEAD_GROUPS + 1][64];
    unsigned long long key[HEAD_GROUPS][DEC_MAX_B];
} DecHeadArrive;

/* Final RMSNorm + LM head + argmax.  Rows: Q8 when wq != NULL, else bf16
 * when wh != NULL, else fp32.  norm_w == NULL: no RMSNorm (a plain
 * out[b][r] = bias[r] + x[b] . W[r], the named fp32/bf16 matmul kernels). */
typedef struct {
    const float* x;      /* [B][D] */
    const float* norm_w;
    const float* bias;   /* [V] added to each output, or NULL */
    const float* w;      /* fp32 [V][D] */
    const unsigned char* wq; /* Q8 [V][D/32] blocks, or NULL */
    const unsigned short* wh; /* 16-bit rows [V][D] (bf16, or IEEE fp16 when wh_f16), or NULL */
    float* logits;       /* [B][V] */
    DecState* st;
    int* out_tokens;     /* [n_gen][B] (generation mode) */
    int D, V, B, tiles;
    float eps;
    int wh_f16;          /* wh holds IEEE fp16 rows (the reference's fp16 precision) */
    DecHeadArrive* arr;  /* the two-level arrival (with st), or NULL: every workgroup at DecState.key and .done */
} DecHead;

/* Every layer of a decode step in one persistent kernel
 * (decode_persist.hip): G instances (1..16; two share each XCD when G > 8),
 * each on one XCD with DEC_PERSIST_WGS working workgroups and NB sequences
 * (1 or 2; instance g runs sequences g NB .. g NB + NB - 1), attention
 * split into nch key chunks per (sequence, KV head) (DEC_PERSIST_NCH at
 * NB = 1), at most DEC_PERSIST_MAX_L layers (the epochs of one step's
 * phases stay below 256).
 *
 * The exchange buffer holds G instance regions of ex_stride 8-byte words.
 * A region carries what its phases pass between workgroups, each float with
 * the epoch of the phase that wrote it (8 bytes: the float's bits in the
 * low word, the epoch in the high word), after three 8-byte words the host
 * never writes:
 *   [0]                   low half, first region only: the step count s
 *                         (advanced by the embedding kernel before every step)
 *   [1, 3)                four 32-bit placement masks: slot s % 4 gathers
 *                         the XCD ids (one bit each) of step s's working
 *                         workgroups of the instance; the persistent kernel
 *                         of step s empties slot (s + 2) % 4 ahead of its
 *                         step, and the host empties all four when the
 *                         kernel is switched on
 *   [3, 3 + NB D)         x, the residual stream after a phase, per sequence
 *   [.., + NB H)          h, the SwiGLU output
 *   [.., + NB (NH*HD + 2 KV))          q, k, v
 *   [.., + NB NH nch (HD+2))           the attention partials (max, sum, P.V[HD])
 *   [.., + NB NH*HD)                   the attention output, merged from the partials */
#define DEC_PERSIST_WGS 32
#define DEC_PERSIST_NCH 10
#ifndef DEC_PERSIST_NCH_B
#define DEC_PERSIST_NCH_B 10 /* most key chunks per (sequence, KV head) at NB = 2 */
#endif
#define DEC_PERSIST_MAX_L 50
#define DEC_PERSIST_EX_HEAD 3 /* 8-byte words before x */
#define DEC_PERSIST_EX_WORDS_NB(D, H, QD, KV, NH, HD, NB, NCH)                                                 \
    (DEC_PERSIST_EX_HEAD + (size_t)(NB) * ((size_t)(D) + (H) + 2 * (size_t)(QD) + 2 * (size_t)(KV) +          \
                                           (size_t)(NH) * (NCH) * ((HD) + 2)))
#define DEC_PERSIST_EX_WORDS(D, H, QD, KV, NH, HD) DEC_PERSIST_EX_WORDS_NB(D, H, QD, KV, NH, HD, 1, DEC_PERSIST_NCH)
typedef struct {
    float* x;                  /* [B][D] residual stream: the embedding at the first layer, the result after the last */
    unsigned long long* ex;    /* the exchange buffer (above), zeroed when allocated */
    float* kvc;                /* the session's KV cache, [B][L][2][MS * KV] */
    DecState* st;
    const unsigned char* w;    /* Q8 arena of layer 0; layer l at w + l * layer_bytes */
    unsigned long long layer_bytes;
    unsigned long long off[7]; /* q, k, v, o, gate, up, down within a layer */
    const float* ln1;          /* [L][D] */
    const float* ln2;          /* [L][D] */
    float inv_freq[DEC_MAX_HD / 2];
    float scale, eps;
    int D, H, NH, NKV, HD, KV, QD, MS, L;
    int NB, G, nch;            /* sequences per instance, instances, key chunks (dec_persist_nch) */
    unsigned long long ex_stride; /* 8-byte words of one instance's exchange region */
    unsigned int spin_ticks;   /* longest wait for an exchanged value, in 100 MHz ticks (0: 0.2 s) */
    int fault_wg;              /* tests only: this working workgroup acts as if on another XCD than its peers (-1: none) */
} DecPersist;

/* Input embedding of a decode step: x[b] = emb[token_b]. */
typedef struct {
    const float* emb;    /* [V][D] */
    const int* prompt;   /* [B][n_prompt] (generation mode) */
    float* x;            /* [B][D] */
    DecState* st;
    unsigned int* steps; /* the persistent step kernel's step counter (advanced here), or NULL */
    int D, V, B;         /* B: the session's batch (one workgroup per sequence) */
} DecEmbed;

#endif
