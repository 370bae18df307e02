/* SPDX-License-Identifier: MPL-2.0
 *
 * engine.cpp — the decode engine behind include/baremetal.h on MI355X.
 *
 * Reference behaviour kept (reference src/baremetal/session.c:34-185,
 * graph.c:109-240, scheduler.c:712-996, tools/run.c:121-185):
 *   per layer  RMSNorm -> q,k,v (Q8) -> RoPE -> KV append + attention over
 *   pos+1 keys -> o (Q8) -> residual add -> RMSNorm -> gate, up (Q8) ->
 *   SwiGLU -> down (Q8) -> residual add; then the final RMSNorm and the LM
 *   head over the tied fp32 embedding; greedy = first maximal logit.
 *
 * MI355X design:
 *   - weights live in HBM: one Q8 arena for every projection (packed on the
 *     device by quantize_q8 from the host fp32 copy), fp32 embedding/head
 *     and norm gains; fp32 KV cache [B][L][2][MS*KV] (K per KV head as [HD/4][MS] float4, V row-major);
 *   - a step is 2 + 5L kernels (embed; per layer: RMSNorm+qkv, rope+KV
 *     append+attention, o+residual, RMSNorm+gate/up+SwiGLU,
 *     down+residual; head+argmax), see decode.hip;
 *   - the position, the input tokens and the argmax live in device memory
 *     (DecState), so the step is captured once into a hipGraph and
 *     replayed; greedy generation runs with no host round trip per token;
 *   - everything is ordered on the backend context's one stream.
 */
#include "bmk.h"
#include "decode_state.h"
#include "q8_gemm.h"
#include "pf_gemm.h"
#include "bm_q8.h"
#include "backend.h"
#include "backend_hip_device.h"
#include "baremetal.h"
#include "bm_synth.h"

#include <math.h>
#include <stdlib.h>
#include <time.h>
#include <string.h>

#include <algorithm>
#include <mutex>
#include <vector>

extern "C" {
int dec_mv_tiles(int OC, int C, int glu);
int dec_head_tiles(int D, int V, int wf);
int dec_launch_embed(const DecEmbed* a, hipStream_t s);
int dec_launch_mv(const DecMv* a, hipStream_t s);
int dec_launch_attn(const DecAttn* a, int B, hipStream_t s);
int dec_pf_embed(const int* tok, const float* emb, float* x, int n, int D, const float* g, unsigned short* an,
                 float* ss, int ss_tiles, int ss_ld, const DecAttn* ra, float* rope, hipStream_t s);
int dec_pf_attention(const DecAttn* a, const float* q, const float* k, const float* v, int n, unsigned short* out16,
                     int kv_done, hipStream_t s);
int q4_pack_f32(const float* src, unsigned char* dst, long n, hipStream_t s);
int q4_pack_bf16(const void* src, unsigned char* dst, long n, hipStream_t s);
int gm_launch_multi_qf(const void* A, int a_bf16, int qf, const unsigned char* W, float* C, const void* plan,
                       int nprob, int n_tiles, hipStream_t s);
int gm_launch_multi(const void* A, int a_bf16, const unsigned char* W, float* C, const void* plan, int nprob,
                    int n_tiles, hipStream_t s);
int gm_cast_bf16(const float* src, unsigned short* dst, long n, hipStream_t s);
int dec_cast_f16(const float* src, unsigned short* dst, long n, hipStream_t s);
int dec_launch_head(const DecHead* a, hipStream_t s);
int dec_persist_ok_b(int D, int H, int NH, int NKV, int HD, int MS, int NB);
int dec_persist_nch(int NKV, int NB);
int dec_persist_hw_ok(const char* arch, int cu_count);
int dec_launch_persist(const DecPersist* a, hipStream_t s);
int q8_pack_f32(const float* src, unsigned char* dst, long n, hipStream_t s);
int q8_pack_bf16(const void* src, unsigned char* dst, long n, hipStream_t s);
}

#define HIP_TRY(call, what, fail)                                                   \
    do {                                                                            \
        hipError_t e_ = (call);                                                     \
        if (e_ != hipSuccess) {                                                     \
            BMK_ERR("%s: %s", what, hipGetErrorString(e_));                         \
            fail;                                                                   \
        }                                                                           \
    } while (0)

struct bm_context_s {
    backend_ctx_t* be;
    hipStream_t s;
};

enum { T_EMB, T_LN1, T_LN2, T_LNF, T_WQ, T_WK, T_WV, T_WO, T_WG, T_WU, T_WD, T_HEAD, T_COUNT };
static const char* const k_tensor_names[T_COUNT] = {"token_embedding", "ln1", "ln2", "lnf", "wq", "wk",
                                                     "wv", "wo", "w_gate", "w_up", "w_down", "lm_head"};

struct bm_model_s {
    bm_context_t* ctx;
    bm_arch_t arch;
    int D, H, NH, NKV, HD, KV, QD, L, V;
    int quant_bits;
    int q8_head;
    bm_precision_t precision; /* BF16: bf16 LM head rows, FP32: fp32 rows */
    float* host[T_COUNT];   /* fp32 weights in the reference layout */
    uint16_t* host16[T_COUNT]; /* bf16 projections as a checkpoint holds them (packed to Q8 from bf16) */
    size_t count[T_COUNT];
    int set[T_COUNT];
    /* device */
    int compiled;
    float* d_emb;
    float* d_ln1;
    float* d_ln2;
    float* d_lnf;
    float* d_headw;          /* untied LM head rows (fp32); NULL when tied */
    unsigned char* d_q8;     /* all projections: per layer q, k, v, o, gate, up, down (Q8_0 or Q4_0 blocks) */
    unsigned char* d_head8;  /* Q8 head rows (q8_head) */
    unsigned short* d_headh; /* 16-bit head rows: bf16 (precision BF16) or fp16 (FP16), no q8_head */
    size_t off[7];           /* byte offset of each matrix inside one layer's slice */
    size_t layer_bytes;
    unsigned char* d_pfw;    /* the same projections in the prefill GEMMs' load order (pf_gemm.h) */
    size_t pf_off[7];        /* byte offset of each matrix inside one layer's slice of d_pfw */
    size_t pf_layer_bytes;
    int nsessions;
};

struct bm_session_s {
    bm_context_t* ctx;
    bm_model_t* m;
    int B, MS;
    float *x, *q, *k, *v, *att, *h, *logits, *kvc;
    /* prefill buffers, allocated on the first bm_forward over a prompt */
    int pf_cap;              /* rows they hold */
    void* pf_buf[9];         /* the prefill workspace (PfWork) */
    DecState* st;
    DecHeadArrive* harr;  /* where the head's workgroups meet (zeroed once, re-armed by every launch) */
    int* prompt;
    int* out_tokens;
    int prompt_cap;
    /* host side */
    DecState* h_st;      /* pinned staging for state writes */
    float* h_logits;     /* pinned [B][V] */
    int* h_io;           /* pinned tokens in/out */
    size_t h_io_cap;
    int pos;             /* host mirror of the position */
    int use_graph;
    int persist;         /* 1: the layers of a step run as one persistent kernel (Q8, MI355X);
                            2: available, per-phase kernels in use; 0: not available */
    int persist_nb, persist_g; /* its sequences per instance and instances (one per XCD) */
    unsigned long long* pex; /* the persistent kernel's exchange buffer (decode_state.h) */
    size_t pex_stride;       /* 8-byte words of one instance's region of it */
    unsigned int persist_spin_ticks; /* tests only: the kernel's longest wait (0: its default) */
    int persist_fault_wg;            /* tests only: a working workgroup that acts as misplaced (-1: none) */
    unsigned long long persist_fallbacks; /* steps rerun on the per-phase kernels after a flagged persistent step */
    hipGraph_t graph;
    hipGraphExec_t gexec;
    int prof_on;
    double prof_ms;
    double prof_phase[BM_PROF_PHASES]; /* ms per phase kind, summed over layers and steps */
    long prof_steps;
    hipEvent_t ev0, ev1;
    double busy_ms;          /* GPU time of host-driven steps and prefills (HIP events) */
    unsigned long long launches; /* step graphs / prefill passes submitted */
    hipEvent_t* pev;     /* one event after every kernel of a profiled step */
    int* pkind;          /* phase kind of the interval that ends at pev[i] */
    int n_pev;
    int mark;            /* next event index while a profiled step is enqueued, -1: not profiling */
};

/* ------------------------------------------------------------------ */
/* context */

extern "C" bm_context_t* bm_create(bm_device_t device) {
    if (device != BM_DEVICE_HIP) {
        BMK_ERR("bm_create: only the GPU device (BM_DEVICE_METAL / BM_DEVICE_HIP) has a backend");
        return NULL;
    }
    backend_ctx_t* be = backend_create();
    if (!be) return NULL;
    bm_context_t* c = (bm_context_t*)calloc(1, sizeof(bm_context_t));
    if (!c) {
        backend_destroy(be);
        return NULL;
    }
    c->be = be;
    c->s = (hipStream_t)be->queue;
    return c;
}

extern "C" void bm_destroy(bm_context_t* ctx) {
    if (!ctx) return;
    backend_destroy(ctx->be);
    free(ctx);
}

extern "C" bm_precision_t bm_get_supported_precision(bm_context_t* ctx) {
    return (ctx && ctx->be && ctx->be->supports_bf16) ? BM_PRECISION_BF16 : BM_PRECISION_FP32;
}

/* ------------------------------------------------------------------ */
/* model */

static size_t q8_bytes(size_t n) { return n / 32 * 36; }

/* Byte offsets of the 7 projections inside one layer's slice of the
 * arena, for the model's block format (Q8_0: 36 bytes, Q4_0: 20 bytes per 32). */
static void layer_layout(bm_model_t* m) {
    const size_t mats[7] = {(size_t)m->QD * m->D, (size_t)m->KV * m->D, (size_t)m->KV * m->D,
                            (size_t)m->D * m->QD, (size_t)m->H * m->D,  (size_t)m->H * m->D,
                            (size_t)m->D * m->H};
    const size_t blk = m->quant_bits == 4 ? 20 : 36;
    size_t o = 0;
    for (int i = 0; i < 7; i++) {
        m->off[i] = o;
        o += mats[i] / 32 * blk;
    }
    m->layer_bytes = o;
    /* the prefill copy: every matrix a whole number of 2304- (1280-) byte chunks */
    const int rows[7] = {m->QD, m->KV, m->KV, m->D, m->H, m->H, m->D};
    const int cols[7] = {m->D, m->D, m->D, m->QD, m->D, m->D, m->H};
    o = 0;
    for (int i = 0; i < 7; i++) {
        m->pf_off[i] = o;
        o += pfg_wbytes(rows[i], cols[i], m->quant_bits == 4);
    }
    m->pf_layer_bytes = o;
}

extern "C" bm_model_t* bm_create_model(bm_context_t* ctx, const bm_arch_t* a) {
    if (!ctx || !a) return NULL;
    const int D = a->dim, H = a->hidden_dim, NH = a->n_heads, NKV = a->n_kv_heads, L = a->n_layers, V = a->vocab_size;
    const int HD = a->head_dim > 0 ? a->head_dim : (NH > 0 ? D / NH : 0);
    if (D <= 0 || H <= 0 || NH <= 0 || NKV <= 0 || L <= 0 || V <= 0 || HD <= 0 || a->max_seq_len <= 0) {
        BMK_ERR("bm_create_model: bad dimensions");
        return NULL;
    }
    if (a->norm != BM_NORM_RMSNORM || a->activation != BM_ACT_SWIGLU || !a->gated_mlp || a->pos_enc != BM_POS_ROPE ||
        a->bias || a->has_qk_norm || a->has_ffn_post_norm || a->gemma_norm || a->embed_scale) {
        BMK_ERR("bm_create_model: only RMSNorm + SwiGLU + RoPE models without biases are supported");
        return NULL;
    }
    if (a->precision != BM_PRECISION_FP32 && a->precision != BM_PRECISION_BF16 && a->precision != BM_PRECISION_FP16) {
        BMK_ERR("bm_create_model: precision %d: the LM head runs in fp32, bf16 or fp16", (int)a->precision);
        return NULL;
    }
    const int QD = NH * HD, KV = NKV * HD;
    /* layout constraints of the gfx950 kernels (decode.hip) */
    if (D % 32 || H % 32 || QD % 32 || D / 32 > 256 || H / 32 > 256 || QD / 32 > 256 || D % 16 || D / 16 > 256 ||
        NH % NKV || HD > 256 || 256 % HD || HD % 4 || KV % 4 || dec_mv_tiles(H, D, 1) < 0) {
        BMK_ERR("bm_create_model: shape D=%d H=%d NH=%d NKV=%d HD=%d outside the decode kernels' layout", D, H, NH, NKV,
                HD);
        return NULL;
    }
    bm_model_t* m = (bm_model_t*)calloc(1, sizeof(bm_model_t));
    if (!m) return NULL;
    m->ctx = ctx;
    m->arch = *a;
    m->D = D; m->H = H; m->NH = NH; m->NKV = NKV; m->HD = HD; m->KV = KV; m->QD = QD; m->L = L; m->V = V;
    m->quant_bits = 8;
    m->precision = a->precision;
    const size_t cnt[T_COUNT] = {(size_t)V * D, (size_t)L * D, (size_t)L * D, (size_t)D, (size_t)L * QD * D,
                                 (size_t)L * KV * D, (size_t)L * KV * D, (size_t)L * D * QD, (size_t)L * H * D,
                                 (size_t)L * H * D, (size_t)L * D * H, a->weight_tie ? 0 : (size_t)V * D};
    memcpy(m->count, cnt, sizeof cnt);
    layer_layout(m);
    return m;
}

static void model_free_device(bm_model_t* m) {
    hipFree(m->d_emb);
    hipFree(m->d_ln1);
    hipFree(m->d_ln2);
    hipFree(m->d_lnf);
    hipFree(m->d_headw);
    m->d_headw = NULL;
    hipFree(m->d_q8);
    hipFree(m->d_pfw);
    m->d_pfw = NULL;
    hipFree(m->d_head8);
    hipFree(m->d_headh);
    m->d_headh = NULL;
    m->d_emb = m->d_ln1 = m->d_ln2 = m->d_lnf = NULL;
    m->d_q8 = m->d_head8 = NULL;
    m->compiled = 0;
}

extern "C" void bm_destroy_model(bm_model_t* m) {
    if (!m) return;
    if (m->ctx) hipStreamSynchronize(m->ctx->s);
    model_free_device(m);
    for (int i = 0; i < T_COUNT; i++) {
        free(m->host[i]);
        free(m->host16[i]);
    }
    free(m);
}

extern "C" int bm_model_set_quant_bits(bm_model_t* m, int bits) {
    if (!m) return -1;
    if (bits != 8 && bits != 4) {
        BMK_ERR("bm_model_set_quant_bits: the MI355X path runs Q8_0 or Q4_0 projections (got %d)", bits);
        return -1;
    }
    if (m->compiled && bits != m->quant_bits) model_free_device(m);
    m->quant_bits = bits;
    layer_layout(m);
    return 0;
}

/* Head rows in use: 1 Q8, 2 bf16, 3 fp16, 0 fp32 (decode.hip's head formats). */
static int head_format(const bm_model_t* m) {
    return m->q8_head ? 1 : m->precision == BM_PRECISION_BF16 ? 2 : m->precision == BM_PRECISION_FP16 ? 3 : 0;
}

extern "C" int bm_model_set_precision(bm_model_t* m, bm_precision_t p) {
    if (!m) return -1;
    if (p != BM_PRECISION_FP32 && p != BM_PRECISION_BF16 && p != BM_PRECISION_FP16) {
        BMK_ERR("bm_model_set_precision: the MI355X path runs the LM head in fp32, bf16 or fp16 (got %d)", (int)p);
        return -1;
    }
    if (m->compiled && p != m->precision) model_free_device(m);
    m->precision = p;
    return 0;
}

extern "C" int bm_model_set_q8_head(bm_model_t* m, int on) {
    if (!m) return -1;
    if (m->compiled && (on != 0) != (m->q8_head != 0)) model_free_device(m);
    m->q8_head = on != 0;
    return 0;
}

static float* host_tensor(bm_model_t* m, int t) {
    if (!m->host[t]) m->host[t] = (float*)malloc(m->count[t] * sizeof(float));
    return m->host[t];
}

static int tensor_index(const bm_model_t* m, const char* name, size_t n, const char* who) {
    for (int t = 0; t < T_COUNT; t++) {
        if (strcmp(name, k_tensor_names[t]) != 0) continue;
        if (m->count[t] == 0) {
            BMK_ERR("%s(%s): the model has no such tensor (tied LM head)", who, name);
            return -1;
        }
        if (n != m->count[t]) {
            BMK_ERR("%s(%s): %zu elements, expected %zu", who, name, n, m->count[t]);
            return -1;
        }
        return t;
    }
    BMK_ERR("%s: unknown tensor %s", who, name);
    return -1;
}

extern "C" int bm_model_set_tensor(bm_model_t* m, const char* name, const float* data, size_t n) {
    if (!m || !name || !data) return -1;
    const int t = tensor_index(m, name, n, "bm_model_set_tensor");
    if (t < 0) return -1;
    float* dst = host_tensor(m, t);
    if (!dst) return -1;
    memcpy(dst, data, n * sizeof(float));
    free(m->host16[t]);
    m->host16[t] = NULL;
    m->set[t] = 1;
    if (m->compiled) model_free_device(m);
    return 0;
}

extern "C" int bm_model_set_tensor_bf16(bm_model_t* m, const char* name, const uint16_t* data, size_t n) {
    if (!m || !name || !data) return -1;
    const int t = tensor_index(m, name, n, "bm_model_set_tensor_bf16");
    if (t < 0) return -1;
    if (t >= T_WQ && t <= T_WD) {
        /* projections stay bf16 until the device packs them */
        if (!m->host16[t]) m->host16[t] = (uint16_t*)malloc(n * sizeof(uint16_t));
        if (!m->host16[t]) return -1;
        memcpy(m->host16[t], data, n * sizeof(uint16_t));
        free(m->host[t]);
        m->host[t] = NULL;
    } else {
        float* dst = host_tensor(m, t);
        if (!dst) return -1;
        for (size_t i = 0; i < n; i++) {
            const uint32_t u = (uint32_t)data[i] << 16; /* exact widening */
            memcpy(dst + i, &u, 4);
        }
    }
    m->set[t] = 1;
    if (m->compiled) model_free_device(m);
    return 0;
}

extern "C" int bm_model_arch(const bm_model_t* m, bm_arch_t* out) {
    if (!m || !out) return -1;
    *out = m->arch;
    return 0;
}

extern "C" int bm_model_init_synthetic(bm_model_t* m, uint64_t seed) {
    if (!m) return -1;
    const size_t per[T_COUNT] = {0, 0, 0, 0, (size_t)m->QD * m->D, (size_t)m->KV * m->D, (size_t)m->KV * m->D,
                                 (size_t)m->D * m->QD, (size_t)m->H * m->D, (size_t)m->H * m->D,
                                 (size_t)m->D * m->H};
    for (int t = 0; t < T_COUNT; t++) {
        if (m->count[t] == 0) continue;
        free(m->host16[t]);
        m->host16[t] = NULL;
        if (!host_tensor(m, t)) return -1;
    }
    bm_synth_normal_f32(bm_synth_tensor_seed(seed, 5, 0xFFFF, 0), 0.02f, m->host[T_EMB], m->count[T_EMB]);
    bm_synth_fill_f32(1.0f, m->host[T_LN1], m->count[T_LN1]);
    bm_synth_fill_f32(1.0f, m->host[T_LN2], m->count[T_LN2]);
    bm_synth_fill_f32(1.0f, m->host[T_LNF], m->count[T_LNF]);
    for (int t = T_WQ; t <= T_WD; t++)
        for (int l = 0; l < m->L; l++)
            bm_synth_normal_f32(bm_synth_tensor_seed(seed, 5, l, t - T_WQ + 1), 0.02f, m->host[t] + (size_t)l * per[t],
                                per[t]);
    if (m->count[T_HEAD]) /* untied: a head of its own, id 8 */
        bm_synth_normal_f32(bm_synth_tensor_seed(seed, 5, 0xFFFF, 8), 0.02f, m->host[T_HEAD], m->count[T_HEAD]);
    for (int t = 0; t < T_COUNT; t++) m->set[t] = 1;
    if (m->compiled) model_free_device(m);
    return 0;
}

static int upload(float** dst, const float* src, size_t n, hipStream_t s) {
    HIP_TRY(hipMalloc(dst, n * sizeof(float)), "hipMalloc", return -1);
    HIP_TRY(hipMemcpyAsync(*dst, src, n * sizeof(float), hipMemcpyHostToDevice, s), "hipMemcpy H2D", return -1);
    return 0;
}

static int model_compile(bm_model_t* m) {
    if (m->compiled) return 0;
    for (int t = 0; t < T_COUNT; t++)
        if (m->count[t] && !m->set[t]) {
            BMK_ERR("bm_compile: tensor %s was never set", k_tensor_names[t]);
            return -1;
        }
    hipStream_t s = m->ctx->s;
    if (upload(&m->d_emb, m->host[T_EMB], m->count[T_EMB], s) || upload(&m->d_ln1, m->host[T_LN1], m->count[T_LN1], s) ||
        upload(&m->d_ln2, m->host[T_LN2], m->count[T_LN2], s) || upload(&m->d_lnf, m->host[T_LNF], m->count[T_LNF], s) ||
        (m->count[T_HEAD] && upload(&m->d_headw, m->host[T_HEAD], m->count[T_HEAD], s))) {
        model_free_device(m);
        return -1;
    }
    const float* head_src = m->d_headw ? m->d_headw : m->d_emb; /* fp32 head rows */
    HIP_TRY(hipMalloc(&m->d_q8, m->layer_bytes * m->L), "hipMalloc", { model_free_device(m); return -1; });
    const int D = m->D, H = m->H, QD = m->QD, KV = m->KV;
    const size_t per[7] = {(size_t)QD * D, (size_t)KV * D, (size_t)KV * D, (size_t)D * QD,
                           (size_t)H * D, (size_t)H * D, (size_t)D * H};
    const int src_t[7] = {T_WQ, T_WK, T_WV, T_WO, T_WG, T_WU, T_WD};
    size_t stage_n = 0; /* the largest matrix staged (q and o are the largest when QD > H) */
    for (int i = 0; i < 7; i++) stage_n = per[i] > stage_n ? per[i] : stage_n;
    if (m->q8_head) stage_n = (size_t)m->V * D > stage_n ? (size_t)m->V * D : stage_n;
    float* stage = NULL;
    HIP_TRY(hipMalloc(&stage, stage_n * sizeof(float)), "hipMalloc", { model_free_device(m); return -1; });
    int rc = 0;
    for (int l = 0; l < m->L && rc == 0; l++)
        for (int i = 0; i < 7 && rc == 0; i++) {
            unsigned char* dst = m->d_q8 + (size_t)l * m->layer_bytes + m->off[i];
            const bool q4 = m->quant_bits == 4;
            if (m->host16[src_t[i]]) { /* bf16 checkpoint: the reference's bmt_quantize_q{8,4}_bf16 on the device */
                const uint16_t* src = m->host16[src_t[i]] + (size_t)l * per[i];
                if (hipMemcpyAsync(stage, src, per[i] * 2, hipMemcpyHostToDevice, s) != hipSuccess) rc = -1;
                else rc = q4 ? q4_pack_bf16(stage, dst, (long)per[i], s) : q8_pack_bf16(stage, dst, (long)per[i], s);
            } else {
                const float* src = m->host[src_t[i]] + (size_t)l * per[i];
                if (hipMemcpyAsync(stage, src, per[i] * sizeof(float), hipMemcpyHostToDevice, s) != hipSuccess) rc = -1;
                else rc = q4 ? q4_pack_f32(stage, dst, (long)per[i], s) : q8_pack_f32(stage, dst, (long)per[i], s);
            }
        }
    /* the prefill's copy of the projections, in its GEMMs' load order */
    if (rc == 0 && hipMalloc(&m->d_pfw, m->pf_layer_bytes * m->L) != hipSuccess) rc = -1;
    for (int l = 0; l < m->L && rc == 0; l++)
        for (int i = 0; i < 7 && rc == 0; i++) {
            const int rows[7] = {QD, KV, KV, D, H, H, D}, cols[7] = {D, D, D, QD, D, D, H};
            rc = pfg_repack(m->d_q8 + (size_t)l * m->layer_bytes + m->off[i],
                            m->d_pfw + (size_t)l * m->pf_layer_bytes + m->pf_off[i], rows[i], cols[i],
                            m->quant_bits == 4, s);
        }
    if (rc == 0 && m->q8_head) {
        if (hipMalloc(&m->d_head8, q8_bytes((size_t)m->V * D)) != hipSuccess) rc = -1;
        else rc = q8_pack_f32(head_src, m->d_head8, (long)m->V * D, s);
    } else if (rc == 0 && head_format(m) >= 2) {
        /* 16-bit rows of the head (the tied embedding or lm_head), rounded to
         * nearest even as the reference's bf16 / fp16 uploads do
         * (scheduler.c:369-374, 395-418) */
        if (hipMalloc(&m->d_headh, (size_t)m->V * D * 2) != hipSuccess) rc = -1;
        else if (head_format(m) == 2) rc = gm_cast_bf16(head_src, m->d_headh, (long)m->V * D, s);
        else rc = dec_cast_f16(head_src, m->d_headh, (long)m->V * D, s);
    }
    if (hipStreamSynchronize(s) != hipSuccess) rc = -1;
    hipFree(stage);
    if (rc != 0) {
        BMK_ERR("bm_compile: weight upload / Q8 pack failed");
        model_free_device(m);
        return -1;
    }
    m->compiled = 1;
    return 0;
}

extern "C" void bm_compile(bm_model_t* m) {
    if (m) (void)model_compile(m);
}

extern "C" int bm_get_num_parameters(const bm_model_t* m) {
    if (!m) return 0;
    size_t n = 0;
    for (int t = 0; t < T_COUNT; t++) n += m->count[t];
    return n > 0x7fffffff ? 0x7fffffff : (int)n;
}

extern "C" const char* bm_get_arch_name(const bm_model_t* m) { return m ? "llama" : NULL; }

/* ------------------------------------------------------------------ */
/* session */

/* Kernel kinds of a step, in launch order within a layer. */
enum { PH_EMBED, PH_QKV, PH_ATTN, PH_O, PH_GATEUP, PH_DOWN, PH_HEAD, PH_LAYERS };

/* Profiled steps: an event after every kernel, tagged with the phase the
 * interval before it belongs to (-1: the step's first event). */
static int mark(bm_session_t* S, int kind) {
    if (S->mark < 0) return 0;
    S->pkind[S->mark] = kind;
    HIP_TRY(hipEventRecord(S->pev[S->mark++], S->ctx->s), "hipEventRecord", return -1);
    return 0;
}

static int enqueue_step(bm_session_t* S) {
    bm_model_t* m = S->m;
    hipStream_t s = S->ctx->s;
    const int D = m->D, B = S->B;
    DecEmbed e;
    e.emb = m->d_emb;
    e.prompt = S->prompt;
    e.x = S->x;
    e.st = S->st;
    e.steps = S->pex ? (unsigned int*)S->pex : NULL;
    e.D = D;
    e.V = m->V;
    e.B = B;
    if (mark(S, -1) || dec_launch_embed(&e, s) || mark(S, PH_EMBED)) return -1;
    const float eps = 1e-5f; /* reference graph.c:134,175,219 */
    if (S->persist == 1) {
        DecPersist pa;
        memset(&pa, 0, sizeof pa);
        pa.x = S->x; pa.ex = S->pex; pa.kvc = S->kvc;
        pa.st = S->st; pa.w = m->d_q8; pa.layer_bytes = m->layer_bytes;
        for (int i = 0; i < 7; i++) pa.off[i] = m->off[i];
        pa.ln1 = m->d_ln1; pa.ln2 = m->d_ln2;
        const float rp[6] = {m->arch.rope_theta, m->arch.rope_factor, m->arch.rope_low_freq_factor,
                             m->arch.rope_high_freq_factor, m->arch.rope_original_max,
                             m->arch.rope_scaling == BM_ROPE_LLAMA3 ? 1.0f : 0.0f};
        bmk_rope_table(rp, m->HD, pa.inv_freq);
        pa.scale = 1.0f / sqrtf((float)m->HD); /* reference scheduler.c:914 */
        pa.eps = eps;
        pa.D = D; pa.H = m->H; pa.NH = m->NH; pa.NKV = m->NKV; pa.HD = m->HD; pa.KV = m->KV; pa.QD = m->QD;
        pa.MS = S->MS; pa.L = m->L;
        pa.NB = S->persist_nb; pa.G = S->persist_g; pa.nch = dec_persist_nch(m->NKV, S->persist_nb);
        pa.ex_stride = S->pex_stride;
        pa.spin_ticks = S->persist_spin_ticks;
        pa.fault_wg = S->persist_fault_wg;
        if (dec_launch_persist(&pa, s) || mark(S, PH_LAYERS)) return -1;
    }
    for (int l = 0; l < (S->persist == 1 ? 0 : m->L); l++) {
        const unsigned char* wl = m->d_q8 + (size_t)l * m->layer_bytes;
        DecMv mv;
        memset(&mv, 0, sizeof mv);
        mv.qf = m->quant_bits == 4;
        DecAttn at;
        memset(&at, 0, sizeof at);
        at.q = S->q; at.k = S->k; at.v = S->v; at.kvc = S->kvc; at.out = S->att; at.st = S->st;
        const float rp[6] = {m->arch.rope_theta, m->arch.rope_factor, m->arch.rope_low_freq_factor,
                             m->arch.rope_high_freq_factor, m->arch.rope_original_max,
                             m->arch.rope_scaling == BM_ROPE_LLAMA3 ? 1.0f : 0.0f};
        bmk_rope_table(rp, m->HD, at.inv_freq);
        at.scale = 1.0f / sqrtf((float)m->HD); /* reference scheduler.c:914 */
        at.NH = m->NH; at.NKV = m->NKV; at.HD = m->HD; at.KV = m->KV; at.MS = S->MS; at.L = m->L; at.layer = l;
        /* RMSNorm + q, k, v */
        mv.x = S->x; mv.norm_w = m->d_ln1 + (size_t)l * D; mv.eps = eps; mv.C = D; mv.B = B; mv.ldx = D;
        mv.nmat = 3;
        mv.w[0] = wl + m->off[0]; mv.y[0] = S->q; mv.OC[0] = m->QD;
        mv.w[1] = wl + m->off[1]; mv.y[1] = S->k; mv.OC[1] = m->KV;
        mv.w[2] = wl + m->off[2]; mv.y[2] = S->v; mv.OC[2] = m->KV;
        mv.tile0[0] = 0;
        for (int i = 0; i < 3; i++) mv.tile0[i + 1] = mv.tile0[i] + dec_mv_tiles(mv.OC[i], D, 0);
        if (dec_launch_mv(&mv, s) || mark(S, PH_QKV)) return -1;
        /* rope + KV append + attention */
        if (dec_launch_attn(&at, B, s) || mark(S, PH_ATTN)) return -1;
        /* o + residual */
        memset(&mv, 0, sizeof mv);
        mv.qf = m->quant_bits == 4;
        mv.x = S->att; mv.C = m->QD; mv.B = B; mv.ldx = m->QD; mv.nmat = 1; mv.residual = 1;
        mv.w[0] = wl + m->off[3]; mv.y[0] = S->x; mv.OC[0] = D;
        mv.tile0[1] = dec_mv_tiles(D, m->QD, 0);
        if (dec_launch_mv(&mv, s) || mark(S, PH_O)) return -1;
        /* RMSNorm + gate, up + SwiGLU */
        memset(&mv, 0, sizeof mv);
        mv.qf = m->quant_bits == 4;
        mv.x = S->x; mv.norm_w = m->d_ln2 + (size_t)l * D; mv.eps = eps; mv.C = D; mv.B = B; mv.ldx = D;
        mv.nmat = 1; mv.glu = 1;
        mv.w[0] = wl + m->off[4]; mv.w[1] = wl + m->off[5]; mv.y[0] = S->h; mv.OC[0] = m->H;
        mv.tile0[1] = dec_mv_tiles(m->H, D, 1);
        if (dec_launch_mv(&mv, s) || mark(S, PH_GATEUP)) return -1;
        /* down + residual */
        memset(&mv, 0, sizeof mv);
        mv.qf = m->quant_bits == 4;
        mv.x = S->h; mv.C = m->H; mv.B = B; mv.ldx = m->H; mv.nmat = 1; mv.residual = 1;
        mv.w[0] = wl + m->off[6]; mv.y[0] = S->x; mv.OC[0] = D;
        mv.tile0[1] = dec_mv_tiles(D, m->H, 0);
        if (dec_launch_mv(&mv, s) || mark(S, PH_DOWN)) return -1;
    }
    DecHead hd;
    memset(&hd, 0, sizeof hd);
    hd.x = S->x; hd.norm_w = m->d_lnf; hd.w = m->d_headw ? m->d_headw : m->d_emb;
    hd.wq = m->q8_head ? m->d_head8 : NULL;
    hd.wh = head_format(m) >= 2 ? m->d_headh : NULL;
    hd.wh_f16 = head_format(m) == 3;
    hd.logits = S->logits; hd.st = S->st; hd.arr = S->harr; hd.out_tokens = S->out_tokens;
    hd.D = D; hd.V = m->V; hd.B = B; hd.eps = eps;
    hd.tiles = dec_head_tiles(D, m->V, head_format(m));
    if (dec_launch_head(&hd, s) || mark(S, PH_HEAD)) return -1;
    return 0;
}

static void session_free(bm_session_t* S) {
    if (!S) return;
    if (S->ctx) hipStreamSynchronize(S->ctx->s);
    if (S->gexec) hipGraphExecDestroy(S->gexec);
    hipFree(S->pex);
    if (S->graph) hipGraphDestroy(S->graph);
    hipFree(S->x); hipFree(S->q); hipFree(S->k); hipFree(S->v); hipFree(S->att); hipFree(S->h);
    hipFree(S->logits); hipFree(S->kvc); hipFree(S->st); hipFree(S->harr); hipFree(S->prompt); hipFree(S->out_tokens);
    for (int i = 0; i < 9; i++) hipFree(S->pf_buf[i]);
    if (S->h_st) hipHostFree(S->h_st);
    if (S->h_logits) hipHostFree(S->h_logits);
    if (S->h_io) hipHostFree(S->h_io);
    if (S->ev0) hipEventDestroy(S->ev0);
    if (S->ev1) hipEventDestroy(S->ev1);
    for (int i = 0; i < S->n_pev; i++) hipEventDestroy(S->pev[i]);
    free(S->pev);
    free(S->pkind);
    if (S->m) S->m->nsessions--;
    free(S);
}

/* Writes the whole DecState from the host (stream-ordered). */
static int state_write(bm_session_t* S) {
    HIP_TRY(hipMemcpyAsync(S->st, S->h_st, sizeof(DecState), hipMemcpyHostToDevice, S->ctx->s), "state write",
            return -1);
    return 0;
}

static int session_reset_state(bm_session_t* S, int host_mode, int n_prompt) {
    memset(S->h_st, 0, sizeof(DecState));
    S->h_st->B = S->B;
    S->h_st->host_mode = host_mode;
    S->h_st->n_prompt = n_prompt;
    S->pos = 0;
    return state_write(S);
}

extern "C" bm_session_t* bm_create_session_batched(bm_context_t* ctx, bm_model_t* m, int batch, int max_seq_len) {
    if (!ctx || !m || m->ctx != ctx) return NULL;
    if (batch < 1 || batch > DEC_MAX_B) {
        BMK_ERR("bm_create_session_batched: batch %d outside [1, %d]", batch, DEC_MAX_B);
        return NULL;
    }
    if (model_compile(m) != 0) return NULL;
    bm_session_t* S = (bm_session_t*)calloc(1, sizeof(bm_session_t));
    if (!S) return NULL;
    S->ctx = ctx;
    S->m = m;
    m->nsessions++;
    S->persist_fault_wg = -1;
    S->B = batch;
    S->MS = max_seq_len > 0 ? max_seq_len : m->arch.max_seq_len;
    S->use_graph = 1;
    S->mark = -1;
    const size_t B = (size_t)batch;
    const size_t kv_elems = B * m->L * 2 * (size_t)S->MS * m->KV;
    bool ok = hipMalloc(&S->x, B * m->D * 4) == hipSuccess && hipMalloc(&S->q, B * m->QD * 4) == hipSuccess &&
              hipMalloc(&S->k, B * m->KV * 4) == hipSuccess && hipMalloc(&S->v, B * m->KV * 4) == hipSuccess &&
              hipMalloc(&S->att, B * m->QD * 4) == hipSuccess && hipMalloc(&S->h, B * m->H * 4) == hipSuccess &&
              hipMalloc(&S->logits, B * m->V * 4) == hipSuccess && hipMalloc(&S->kvc, kv_elems * 4) == hipSuccess &&
              hipMalloc(&S->st, sizeof(DecState)) == hipSuccess &&
              hipMalloc(&S->harr, sizeof(DecHeadArrive)) == hipSuccess &&
              hipMemsetAsync(S->harr, 0, sizeof(DecHeadArrive), ctx->s) == hipSuccess &&
              hipMalloc(&S->out_tokens, B * (size_t)S->MS * 4) == hipSuccess &&
              hipMalloc(&S->prompt, B * (size_t)S->MS * 4) == hipSuccess &&

              hipHostMalloc(&S->h_st, sizeof(DecState), hipHostMallocDefault) == hipSuccess &&
              hipHostMalloc(&S->h_logits, B * m->V * 4, hipHostMallocDefault) == hipSuccess &&
              hipEventCreate(&S->ev0) == hipSuccess && hipEventCreate(&S->ev1) == hipSuccess;
    if (ok) {
        S->prompt_cap = S->MS;
        S->h_io_cap = B * (size_t)S->MS + 64;
        ok = hipHostMalloc(&S->h_io, S->h_io_cap * 4, hipHostMallocDefault) == hipSuccess;
    }
    /* The persistent step kernel runs instances of 32 workgroups, each
     * keeping its workgroups on one XCD (MI355X places workgroup b on XCD
     * (b + start) % 8): up to 16 sequences one per instance, 32 two per
     * instance, with two instances per XCD past 8.  Only where the device
     * fits its memory-model assumptions (dec_persist_hw_ok), with Q8
     * projections and a shape it handles (dec_persist_ok_b, which also
     * checks the conditions its buffer reuse relies on). */
    int nb = batch <= 16 ? 1 : (batch <= 32 && batch % 2 == 0) ? 2 : 0;
    if (ok && nb && m->quant_bits == 8 && dec_persist_hw_ok(ctx->be->dev_name, ctx->be->dev_cu_count) &&
        m->L <= DEC_PERSIST_MAX_L && dec_persist_ok_b(m->D, m->H, m->NH, m->NKV, m->HD, S->MS, nb)) {
        S->persist_nb = nb;
        S->persist_g = batch / nb;
        /* instance regions start on 256-byte lines */
        S->pex_stride = (DEC_PERSIST_EX_WORDS_NB(m->D, m->H, m->QD, m->KV, m->NH, m->HD, nb,
                                                 dec_persist_nch(m->NKV, nb)) + 31) & ~(size_t)31;
        const size_t ex = S->pex_stride * S->persist_g * 8;
        ok = hipMalloc(&S->pex, ex) == hipSuccess && hipMemsetAsync(S->pex, 0, ex, ctx->s) == hipSuccess;
        S->persist = ok;
    }
    /* a cache slot is written before it is read, but start from zeros anyway */
    if (ok) ok = hipMemsetAsync(S->kvc, 0, kv_elems * 4, ctx->s) == hipSuccess;
    if (ok) ok = session_reset_state(S, 1, 0) == 0;
    if (ok) ok = hipStreamSynchronize(ctx->s) == hipSuccess;
    if (!ok) {
        (void)hipGetLastError();
        BMK_ERR("bm_create_session: device allocation failed");
        session_free(S);
        return NULL;
    }
    return S;
}

extern "C" bm_session_t* bm_create_session(bm_context_t* ctx, bm_model_t* m) {
    return bm_create_session_batched(ctx, m, 1, 0);
}

extern "C" void bm_destroy_session(bm_session_t* S) { session_free(S); }

extern "C" int bm_session_set_graph(bm_session_t* S, int on) {
    if (!S) return -1;
    S->use_graph = on != 0;
    return 0;
}

extern "C" int bm_session_set_persistent(bm_session_t* S, int on) {
    if (!S) return -1;
    if (S->persist == 0) return on ? -1 : 0; /* not available for this session */
    const int want = on ? 1 : 2;
    if (S->persist != want && S->gexec) { /* the captured step is the other form */
        hipGraphExecDestroy(S->gexec);
        hipGraphDestroy(S->graph);
        S->gexec = NULL;
        S->graph = NULL;
    }
    /* switched back on: the kernel empties each step's placement slot two
     * steps ahead only while it runs, so all four start empty again */
    if (S->persist == 2 && want == 1)
        for (int g = 0; g < S->persist_g; g++)
            HIP_TRY(hipMemsetAsync(S->pex + g * S->pex_stride + 1, 0, 16, S->ctx->s), "placement slots", return -1);
    S->persist = want;
    return 0;
}

/* Tests only: forces the persistent step kernel's failure paths from the
 * host, every kernel still exiting normally.  mode 1: every wait for an
 * exchanged value gives up after one 100 MHz tick (as a timeout would);
 * mode 2: working workgroup 5 acts as if on another XCD than its peers; mode 0: neither.
 * Drops a captured step (its arguments change).  Returns the session's
 * persistent state (0 not available, 1 in use, 2 per-phase kernels in use)
 * and, in *fallbacks, how many steps were rerun on the per-phase kernels. */
extern "C" int bm_session_persist_test_fault(bm_session_t* S, int mode, unsigned long long* fallbacks) {
    if (!S || mode < 0 || mode > 2) return -1;
    S->persist_spin_ticks = mode == 1 ? 1u : 0u;
    S->persist_fault_wg = mode == 2 ? 5 : -1;
    if (S->gexec) {
        hipGraphExecDestroy(S->gexec);
        hipGraphDestroy(S->graph);
        S->gexec = NULL;
        S->graph = NULL;
    }
    if (fallbacks) *fallbacks = S->persist_fallbacks;
    return S->persist;
}

static int ensure_graph(bm_session_t* S) {
    if (S->gexec) return 0;
    hipStream_t s = S->ctx->s;
    HIP_TRY(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal), "hipStreamBeginCapture", return -1);
    const int rc = enqueue_step(S);
    hipGraph_t g = NULL;
    hipError_t e = hipStreamEndCapture(s, &g);
    if (rc != 0 || e != hipSuccess) {
        BMK_ERR("step capture failed: %s", hipGetErrorString(e));
        if (g) hipGraphDestroy(g);
        (void)hipGetLastError();
        return -1;
    }
    HIP_TRY(hipGraphInstantiate(&S->gexec, g, NULL, NULL, 0), "hipGraphInstantiate", {
        hipGraphDestroy(g);
        return -1;
    });
    S->graph = g;
    return 0;
}

static int launch_step(bm_session_t* S) {
    if (S->pos >= S->MS) {
        BMK_ERR("decode step: position %d reached max_seq_len %d", S->pos, S->MS);
        return -1;
    }
    if (S->prof_on) {
        /* profiled steps run eagerly with an event after every kernel */
        const int need = 3 + 5 * S->m->L;
        if (S->n_pev < need) {
            hipEvent_t* ev = (hipEvent_t*)realloc(S->pev, (size_t)need * sizeof(hipEvent_t));
            if (!ev) return -1;
            S->pev = ev;
            int* pk = (int*)realloc(S->pkind, (size_t)need * sizeof(int));
            if (!pk) return -1;
            S->pkind = pk;
            for (; S->n_pev < need; S->n_pev++)
                HIP_TRY(hipEventCreate(&S->pev[S->n_pev]), "hipEventCreate", return -1);
        }
        S->mark = 0;
        const int rc = enqueue_step(S);
        const int n = S->mark;
        S->mark = -1;
        if (rc != 0) return -1;
        HIP_TRY(hipEventSynchronize(S->pev[n - 1]), "hipEventSynchronize", return -1);
        float ms = 0.f;
        if (hipEventElapsedTime(&ms, S->pev[0], S->pev[n - 1]) == hipSuccess) S->prof_ms += ms;
        for (int i = 1; i < n; i++) {
            const int kind = S->pkind[i];
            if (kind >= 0 && hipEventElapsedTime(&ms, S->pev[i - 1], S->pev[i]) == hipSuccess)
                S->prof_phase[kind] += ms;
        }
        S->prof_steps++;
    } else if (S->use_graph) {
        if (ensure_graph(S) != 0) return -1;
        HIP_TRY(hipGraphLaunch(S->gexec, S->ctx->s), "hipGraphLaunch", return -1);
    } else if (enqueue_step(S) != 0) {
        return -1;
    }
    S->pos++;
    return 0;
}

/* A persistent step flagged void (DecState.sync_error: a wait timed out, or
 * a workgroup ran on another XCD than its peers): the session switches to the per-phase
 * kernels for good, and the device state goes back to what it was before
 * the step (position, no error), so the step can run again.  What the
 * flagged step wrote is rewritten by the rerun: the embedding, every
 * layer's KV slot at the step's position and the head's outputs; the head
 * re-arms its argmax keys and arrival counter itself. */
static int persist_fallback(bm_session_t* S, int pos) {
    BMK_ERR("decode step: the persistent step kernel flagged step %d void (sync_error %d: %s); rerunning it, and "
            "every later step, on the per-phase kernels",
            pos, S->h_st->sync_error, S->h_st->sync_error == 2 ? "a workgroup ran on another XCD than its peers" : "a wait timed out");
    if (bm_session_set_persistent(S, 0) != 0) return -1;
    S->persist_fallbacks++;
    S->h_st->sync_error = 0;
    S->pos = pos;
    int* w = &S->h_io[S->B + 1]; /* pinned staging past the tokens and the mode word */
    w[0] = pos;
    w[1] = 0;
    HIP_TRY(hipMemcpyAsync(&S->st->pos, &w[0], 4, hipMemcpyHostToDevice, S->ctx->s), "state write", return -1);
    HIP_TRY(hipMemcpyAsync(&S->st->sync_error, &w[1], 4, hipMemcpyHostToDevice, S->ctx->s), "state write", return -1);
    return 0;
}

/* Host-driven step: tokens[b] in, logits [B][V] back to the host. */
static float* step_host(bm_session_t* S, const int* tokens) {
    bm_model_t* m = S->m;
    for (int b = 0; b < S->B; b++)
        if (tokens[b] < 0 || tokens[b] >= m->V) {
            BMK_ERR("bm_step: token %d outside [0, %d)", tokens[b], m->V);
            return NULL;
        }
    if (!S->h_st->host_mode) { /* leaving generation mode: keep the position */
        S->h_st->host_mode = 1;
    }
    HIP_TRY(hipStreamSynchronize(S->ctx->s), "sync", return NULL);
    memcpy(S->h_io, tokens, (size_t)S->B * 4);
    HIP_TRY(hipMemcpyAsync(S->st->host_token, S->h_io, (size_t)S->B * 4, hipMemcpyHostToDevice, S->ctx->s),
            "token write", return NULL);
    const int one = 1;
    memcpy(&S->h_io[S->B], &one, 4);
    HIP_TRY(hipMemcpyAsync(&S->st->host_mode, &S->h_io[S->B], 4, hipMemcpyHostToDevice, S->ctx->s), "mode write",
            return NULL);
    const int pos = S->pos;
    for (;;) {
        const bool persistent = S->persist == 1;
        HIP_TRY(hipEventRecord(S->ev0, S->ctx->s), "event", return NULL);
        if (launch_step(S) != 0) return NULL;
        HIP_TRY(hipEventRecord(S->ev1, S->ctx->s), "event", return NULL);
        HIP_TRY(hipMemcpyAsync(S->h_logits, S->logits, (size_t)S->B * m->V * 4, hipMemcpyDeviceToHost, S->ctx->s),
                "logits read", return NULL);
        if (persistent)
            HIP_TRY(hipMemcpyAsync(&S->h_st->sync_error, &S->st->sync_error, 4, hipMemcpyDeviceToHost, S->ctx->s),
                    "state read", return NULL);
        HIP_TRY(hipStreamSynchronize(S->ctx->s), "sync", return NULL);
        if (!persistent || !S->h_st->sync_error) break;
        if (persist_fallback(S, pos) != 0) return NULL; /* then once more on the per-phase kernels */
    }
    float ms = 0.f;
    if (hipEventElapsedTime(&ms, S->ev0, S->ev1) == hipSuccess) S->busy_ms += ms;
    S->launches++;
    return S->h_logits;
}

extern "C" float* bm_step(bm_session_t* S, int token) {
    if (!S) return NULL;
    if (S->B != 1) {
        BMK_ERR("bm_step: batched session, use bm_step_batch");
        return NULL;
    }
    return step_host(S, &token);
}

extern "C" float* bm_step_batch(bm_session_t* S, const int* tokens) {
    if (!S || !tokens) return NULL;
    return step_host(S, tokens);
}

/* ------------------------------------------------------------------ */
/* prefill: a whole prompt at position 0 (reference session.c:86-139) */

/* The prefill's workspace for n tokens: the residual stream x [n][D], the
 * q/k/v rows, the attention output (fp32, head sizes other than 64), the
 * bf16 GEMM operands in MFMA fragment order (rows rounded up to 32, columns
 * to 64): a16 for the first RMSNorm's and the attention's outputs, h16 for
 * the SwiGLU output, a16b for the second RMSNorm's; the tokens, the RoPE
 * (cos, sin) table of the prompt's positions, and the rows' partial sums of
 * squares [2 ceil(D / 64)][n] for the RMSNorm scale (one per column tile of
 * the residual GEMM that wrote them: its 32-column tiles cover whole
 * 64-column steps).  bm_forward keeps it in session buffers allocated
 * on the first prefill; bm_forward_noalloc carves it from the library's
 * static per-GPU array. */
struct PfWork {
    float *x, *qkv, *att;
    unsigned short *a16, *h16;
    int* tok;
    float* rope;
    unsigned short* a16b;
    float* ss;
};

#define PF_PARTS 9

/* Device bytes of each part for n tokens (sz), and their offsets in one
 * 256-aligned carve (off, when given); returns the total. */
static size_t pf_work_layout(const bm_model_t* m, int n, size_t sz[PF_PARTS], size_t off[PF_PARTS]) {
    const size_t N = (size_t)n, N32 = (N + 31) / 32 * 32;
    const size_t a_cols = ((size_t)std::max(m->D, m->QD) + 63) / 64 * 64, h_cols = ((size_t)m->H + 63) / 64 * 64;
    const size_t b[PF_PARTS] = {N * m->D * 4, N * (m->QD + 2 * (size_t)m->KV) * 4, N * m->QD * 4, N32 * a_cols * 2,
                                N32 * h_cols * 2, N * 4, N * (size_t)(m->HD / 2) * 8,
                                N32 * (((size_t)m->D + 63) / 64 * 64) * 2, ((size_t)m->D + 63) / 64 * 2 * N * 4};
    size_t at = 0;
    for (int i = 0; i < PF_PARTS; i++) {
        if (sz) sz[i] = b[i];
        if (off) off[i] = at;
        at += (b[i] + 255) & ~(size_t)255;
    }
    return at;
}

static void pf_work_set(PfWork* w, void* const part[PF_PARTS]) {
    w->x = (float*)part[0]; w->qkv = (float*)part[1]; w->att = (float*)part[2];
    w->a16 = (unsigned short*)part[3]; w->h16 = (unsigned short*)part[4]; w->tok = (int*)part[5];
    w->rope = (float*)part[6]; w->a16b = (unsigned short*)part[7]; w->ss = (float*)part[8];
}

/* bm_forward's workspace: session buffers, grown to n tokens. */
static int pf_session_work(bm_session_t* S, int n, PfWork* w) {
    if (S->pf_cap < n) {
        for (int i = 0; i < PF_PARTS; i++) {
            hipFree(S->pf_buf[i]);
            S->pf_buf[i] = NULL;
        }
        S->pf_cap = 0;
        size_t sz[PF_PARTS];
        pf_work_layout(S->m, n, sz, NULL);
        for (int i = 0; i < PF_PARTS; i++)
            if (hipMalloc(&S->pf_buf[i], sz[i]) != hipSuccess) {
                (void)hipGetLastError();
                BMK_ERR("bm_forward: prefill buffers for %d tokens could not be allocated", n);
                return -1;
            }
        S->pf_cap = n;
    }
    pf_work_set(w, S->pf_buf);
    return 0;
}

extern "C" void* bmk_noalloc_scratch(int device);

/* Each GPU's static array is shared by every bm_forward_noalloc call on that
 * GPU, so s_noalloc_mu serializes the calls: it is held from the workspace
 * carve to the final synchronization on the logits read. */
static std::mutex s_noalloc_mu;

/* bm_forward_noalloc's workspace: carved from the GPU's static array; -1
 * (logged) when n tokens do not fit. */
static int pf_noalloc_work(bm_session_t* S, int n, PfWork* w) {
    const int dev = (int)(intptr_t)S->ctx->be->device;
    unsigned char* base = (unsigned char*)bmk_noalloc_scratch(dev);
    if (!base) return -1;
    size_t off[PF_PARTS];
    const size_t act = pf_work_layout(S->m, n, NULL, off);
    if (act > BM_NOALLOC_SCRATCH_BYTES) {
        BMK_ERR("bm_forward_noalloc: %d tokens need %zu workspace bytes, the static array holds %u", n, act,
                (unsigned)BM_NOALLOC_SCRATCH_BYTES);
        return -1;
    }
    void* part[PF_PARTS];
    for (int i = 0; i < PF_PARTS; i++) part[i] = base + off[i];
    pf_work_set(w, part);
    return 0;
}

static int prefill(bm_session_t* S, const int* tokens, int n, bool noalloc) {
    bm_model_t* m = S->m;
    hipStream_t s = S->ctx->s;
    const int D = m->D, H = m->H, QD = m->QD, KV = m->KV, L = m->L;
    const float eps = 1e-5f; /* reference graph.c:134,175,219 */
    for (int i = 0; i < n; i++)
        if (tokens[i] < 0 || tokens[i] >= m->V) {
            BMK_ERR("bm_forward: token %d outside [0, %d)", tokens[i], m->V);
            return -1;
        }
    PfWork w;
    HIP_TRY(hipStreamSynchronize(s), "sync", return -1); /* the token staging buffer may still be read */
    if ((noalloc ? pf_noalloc_work(S, n, &w) : pf_session_work(S, n, &w)) != 0) return -1;
    memcpy(S->h_io, tokens, (size_t)n * 4);
    HIP_TRY(hipMemcpyAsync(w.tok, S->h_io, (size_t)n * 4, hipMemcpyHostToDevice, s), "token write", return -1);

    DecAttn at;
    memset(&at, 0, sizeof at);
    at.kvc = S->kvc;
    at.out = w.att;
    const float rp[6] = {m->arch.rope_theta, m->arch.rope_factor, m->arch.rope_low_freq_factor,
                         m->arch.rope_high_freq_factor, m->arch.rope_original_max,
                         m->arch.rope_scaling == BM_ROPE_LLAMA3 ? 1.0f : 0.0f};
    bmk_rope_table(rp, m->HD, at.inv_freq);
    at.scale = 1.0f / sqrtf((float)m->HD); /* reference scheduler.c:914 */
    at.NH = m->NH; at.NKV = m->NKV; at.HD = m->HD; at.KV = KV; at.MS = S->MS; at.L = L;

    float* q = w.qkv;
    float* k = q + (size_t)n * QD;
    float* v = k + (size_t)n * KV;
    const int qf = m->quant_bits == 4;
    /* head size 64: RoPE and the cache append run in the q/k/v GEMM's epilogue */
    const int kv_fused = m->HD == 64;
    const size_t slab = (size_t)S->MS * KV;
    /* RMSNorm runs in the launches around it: the embedding and each
     * residual GEMM write bf16(x * g) of the next norm and the rows' partial
     * sums of squares, and the GEMM that takes them scales its rows */
    int ss_parts = 1; /* the partial sums per row the last writer left (the embedding: the whole sum) */
    if (dec_pf_embed(w.tok, m->d_emb, w.x, n, D, m->d_ln1, w.a16, w.ss, ss_parts, n, &at, kv_fused ? w.rope : NULL,
                     s))
        return -1;
    for (int l = 0; l < L; l++) {
        at.layer = l;
        const uint64_t lw = (uint64_t)l * m->pf_layer_bytes;
        PfgArgs qkv, o, gu, dn;
        memset(&qkv, 0, sizeof qkv);
        qkv.A = w.a16; qkv.W = m->d_pfw; qkv.M = n; qkv.K = D; qkv.nprob = 3;
        qkv.p[0].w_off = lw + m->pf_off[0]; qkv.p[0].C = q; qkv.p[0].N = QD; qkv.p[0].ldc = QD;
        qkv.p[1].w_off = lw + m->pf_off[1]; qkv.p[1].C = k; qkv.p[1].N = KV; qkv.p[1].ldc = KV;
        qkv.p[2].w_off = lw + m->pf_off[2]; qkv.p[2].C = v; qkv.p[2].N = KV; qkv.p[2].ldc = KV;
        qkv.ss_in = w.ss; qkv.ss_tiles = ss_parts; qkv.ss_ld = n; qkv.norm_d = D; qkv.eps = eps;
        if (kv_fused) {
            qkv.kc = S->kvc + (size_t)l * 2 * slab;
            qkv.vc = qkv.kc + slab;
            qkv.MS = S->MS;
            qkv.rope = w.rope;
        }
        memset(&o, 0, sizeof o);
        o.A = w.a16; o.W = m->d_pfw; o.x = w.x; o.M = n; o.K = QD; o.nprob = 1;
        o.p[0].w_off = lw + m->pf_off[3]; o.p[0].N = D; o.p[0].ldc = D;
        o.an = w.a16b; o.gn = m->d_ln2 + (size_t)l * D; o.ss_out = w.ss; o.ss_ld = n;
        memset(&gu, 0, sizeof gu);
        gu.A = w.a16b; gu.W = m->d_pfw; gu.h = w.h16; gu.M = n; gu.K = D; gu.nprob = 2;
        gu.p[0].w_off = lw + m->pf_off[4]; gu.p[0].N = H;
        gu.p[1].w_off = lw + m->pf_off[5]; gu.p[1].N = H;
        gu.ss_in = w.ss; gu.ss_ld = n; gu.norm_d = D; gu.eps = eps;
        memset(&dn, 0, sizeof dn);
        dn.A = w.h16; dn.W = m->d_pfw; dn.x = w.x; dn.M = n; dn.K = H; dn.nprob = 1;
        dn.p[0].w_off = lw + m->pf_off[6]; dn.p[0].N = D; dn.p[0].ldc = D;
        if (l + 1 < L) {
            dn.an = w.a16; dn.gn = m->d_ln1 + (size_t)(l + 1) * D; dn.ss_out = w.ss; dn.ss_ld = n;
        }
        /* q/k/v (RMSNorm 1); RoPE, cache append, causal attention; o + residual
         * (RMSNorm 2's operand); gate/up + SwiGLU; down + residual (the next
         * layer's RMSNorm 1 operand) */
        if (pfg_launch(&qkv, qf, kv_fused ? PFG_QKV : PFG_STORE, s) ||
            dec_pf_attention(&at, q, k, v, n, w.a16, kv_fused, s) ||
            pfg_launch(&o, qf, PFG_RESID, s))
            return -1;
        gu.ss_tiles = o.NT; /* the o launch's column tiles */
        if (pfg_launch(&gu, qf, PFG_SWIGLU, s) || pfg_launch(&dn, qf, PFG_RESID, s)) return -1;
        ss_parts = dn.NT;
    }
    /* the head on the last position (its own final RMSNorm) */
    DecHead hd;
    memset(&hd, 0, sizeof hd);
    hd.x = w.x + (size_t)(n - 1) * D; hd.norm_w = m->d_lnf; hd.w = m->d_headw ? m->d_headw : m->d_emb;
    hd.wq = m->q8_head ? m->d_head8 : NULL;
    hd.wh = head_format(m) >= 2 ? m->d_headh : NULL;
    hd.wh_f16 = head_format(m) == 3;
    hd.logits = S->logits; hd.st = NULL; hd.out_tokens = NULL;
    hd.D = D; hd.V = m->V; hd.B = 1; hd.eps = eps;
    hd.tiles = dec_head_tiles(D, m->V, head_format(m));
    if (dec_launch_head(&hd, s)) return -1;
    /* the decode steps continue at position n */
    memset(S->h_st, 0, sizeof(DecState));
    S->h_st->B = S->B;
    S->h_st->host_mode = 1;
    S->h_st->pos = n;
    if (state_write(S)) return -1;
    HIP_TRY(hipMemcpyAsync(S->h_logits, S->logits, (size_t)m->V * 4, hipMemcpyDeviceToHost, s), "logits read",
            return -1);
    HIP_TRY(hipStreamSynchronize(s), "sync", return -1);
    S->pos = n;
    return 0;
}

/* One timed one-pass prefill (the session is at position 0, batch 1). */
static float* forward_prefill(bm_session_t* S, const int* tokens, int n_tokens, bool noalloc) {
    HIP_TRY(hipStreamSynchronize(S->ctx->s), "sync", return NULL);
    HIP_TRY(hipEventRecord(S->ev0, S->ctx->s), "event", return NULL);
    if (prefill(S, tokens, n_tokens, noalloc) != 0) return NULL;
    float ms = 0.f;
    /* prefill ends synchronized on the logits read: ev0 to now is its GPU span */
    if (hipEventRecord(S->ev1, S->ctx->s) == hipSuccess && hipEventSynchronize(S->ev1) == hipSuccess &&
        hipEventElapsedTime(&ms, S->ev0, S->ev1) == hipSuccess)
        S->busy_ms += ms;
    S->launches++;
    return S->h_logits;
}

/* Reference session.c:141-149: a prompt at position 0 of a batch-1 session
 * is prefilled in one pass (bf16-MFMA projections); anything else steps
 * token by token. */
extern "C" float* bm_forward(bm_session_t* S, const int* tokens, int n_tokens) {
    if (!S || (!tokens && n_tokens > 0)) return NULL;
    if (n_tokens <= 0) return S->h_logits;
    if (n_tokens > 1 && S->pos == 0 && S->B == 1 && n_tokens <= S->MS && (size_t)n_tokens <= S->h_io_cap)
        return forward_prefill(S, tokens, n_tokens, false);
    float* out = S->h_logits;
    for (int i = 0; i < n_tokens; i++) {
        out = bm_step(S, tokens[i]);
        if (!out) return NULL;
    }
    return out;
}

/* bm_forward's one-pass prefill with its workspace in the library's static
 * per-GPU array (include/baremetal.h): no allocation of any kind. */
extern "C" float* bm_forward_noalloc(bm_session_t* S, const int* tokens, int n_tokens) {
    if (!S || !tokens || n_tokens < 2) {
        BMK_ERR("bm_forward_noalloc: needs a session and at least 2 tokens (got %d)", n_tokens);
        return NULL;
    }
    if (S->pos != 0 || S->B != 1 || n_tokens > S->MS || (size_t)n_tokens > S->h_io_cap) {
        BMK_ERR("bm_forward_noalloc: a prompt of %d tokens at position 0 of a batch-1 session with room for it "
                "(position %d, batch %d, max %d)", n_tokens, S->pos, S->B, S->MS);
        return NULL;
    }
    std::lock_guard<std::mutex> lock(s_noalloc_mu);
    return forward_prefill(S, tokens, n_tokens, true);
}

extern "C" int bm_session_gpu_stats(bm_session_t* S, double* busy_ms, unsigned long long* launches, int reset) {
    if (!S) return -1;
    if (busy_ms) *busy_ms = S->busy_ms;
    if (launches) *launches = S->launches;
    if (reset) {
        S->busy_ms = 0.0;
        S->launches = 0;
    }
    return 0;
}

extern "C" void bm_reset_session(bm_session_t* S) {
    if (!S) return;
    hipStreamSynchronize(S->ctx->s);
    session_reset_state(S, 1, 0);
    hipStreamSynchronize(S->ctx->s);
}

extern "C" int bm_generate_greedy(bm_session_t* S, const int* prompt, int n_prompt, int steps, int* out_tokens) {
    if (!S || !prompt || !out_tokens || n_prompt < 1 || steps < n_prompt || steps > S->MS || n_prompt > S->prompt_cap) {
        BMK_ERR("bm_generate_greedy: bad arguments (n_prompt=%d steps=%d max_seq_len=%d)", n_prompt, steps, S ? S->MS : 0);
        return -1;
    }
    const size_t np = (size_t)S->B * n_prompt;
    for (size_t i = 0; i < np; i++)
        if (prompt[i] < 0 || prompt[i] >= S->m->V) {
            BMK_ERR("bm_generate_greedy: prompt token %d outside [0, %d)", prompt[i], S->m->V);
            return -1;
        }
    HIP_TRY(hipStreamSynchronize(S->ctx->s), "sync", return -1);
    memcpy(S->h_io, prompt, np * 4);
    HIP_TRY(hipMemcpyAsync(S->prompt, S->h_io, np * 4, hipMemcpyHostToDevice, S->ctx->s), "prompt write", return -1);
    const int n_out = steps - n_prompt + 1;
    const size_t nt = (size_t)n_out * S->B;
    for (;;) {
        const bool persistent = S->persist == 1;
        if (session_reset_state(S, 0, n_prompt) != 0) return -1;
        for (int i = 0; i < steps; i++)
            if (launch_step(S) != 0) return -1;
        HIP_TRY(hipMemcpyAsync(S->h_io, S->out_tokens, nt * 4, hipMemcpyDeviceToHost, S->ctx->s), "tokens read",
                return -1);
        HIP_TRY(hipMemcpyAsync(S->h_st, S->st, sizeof(DecState), hipMemcpyDeviceToHost, S->ctx->s), "state read",
                return -1);
        HIP_TRY(hipStreamSynchronize(S->ctx->s), "sync", return -1);
        /* a flagged persistent step voids the run (every later step gives up
         * at once): the whole run again on the per-phase kernels */
        if (!persistent || !S->h_st->sync_error) break;
        if (persist_fallback(S, 0) != 0) return -1;
    }
    if (S->h_st->n_out != n_out || S->h_st->pos != steps || S->h_st->bad_token || S->h_st->sync_error) {
        BMK_ERR("bm_generate_greedy: device state n_out=%d pos=%d bad_token=%d sync_error=%d, expected n_out=%d pos=%d",
                S->h_st->n_out, S->h_st->pos, S->h_st->bad_token, S->h_st->sync_error, n_out, steps);
        return -1;
    }
    memcpy(out_tokens, S->h_io, nt * 4);
    return n_out;
}

extern "C" void bm_profile_begin(bm_session_t* S) {
    if (!S) return;
    S->prof_on = 1;
    S->prof_ms = 0.0;
    S->prof_steps = 0;
    for (int i = 0; i < BM_PROF_PHASES; i++) S->prof_phase[i] = 0.0;
}

extern "C" void bm_profile_end(bm_session_t* S, double* attention_ms, double* mlp_ms, double* other_ms) {
    const double* p = S ? S->prof_phase : NULL;
    if (attention_ms) *attention_ms = p ? p[PH_QKV] + p[PH_ATTN] + p[PH_O] : 0.0;
    if (mlp_ms) *mlp_ms = p ? p[PH_GATEUP] + p[PH_DOWN] : 0.0;
    if (other_ms) *other_ms = p ? p[PH_EMBED] + p[PH_HEAD] : 0.0;
    if (S) S->prof_on = 0;
}

extern "C" long bm_profile_phases(bm_session_t* S, double* ms) {
    if (!S || !ms) return -1;
    for (int i = 0; i < BM_PROF_PHASES; i++) ms[i] = S->prof_phase[i];
    return S->prof_steps;
}

/* ------------------------------------------------------------------ */
/* sampler: reference src/baremetal/sampler.c:33-81 (bm_sample) and
 * tools/run.c:53-104 (the driver's draw).  Both run temperature -> softmax
 * -> top-k mask -> top-p mask -> one hashed-LCG draw over the cumulative
 * sum; they differ in three places, kept here as the reference has them:
 * bm_sample's sampler starts with top_k = 40 (reference api.c:85), chains
 * its state (the hash output becomes the next state, sampler.c:74-76) and
 * returns n - 1 when the cumulative sum never reaches the target
 * (sampler.c:80); the driver hashes seed, seed + 1, ... (run.c:172) and
 * returns 0 there (run.c:100). */

struct bm_sampler_s {
    int vocab_size;
    float temperature;
    float topp;
    int top_k;
    unsigned int rng;
    float* probs;
    float* sorted; /* scratch: the probabilities in descending order */
};

extern "C" bm_sampler_t* bm_create_sampler(int vocab_size, float temp, float topp, uint64_t seed) {
    if (vocab_size <= 0) return NULL;
    bm_sampler_t* s = (bm_sampler_t*)calloc(1, sizeof(bm_sampler_t));
    if (!s) return NULL;
    s->vocab_size = vocab_size;
    s->temperature = temp;
    s->topp = topp;
    s->top_k = 40;
    s->rng = (unsigned int)seed;
    if (seed == 0) s->rng = (unsigned int)(uintptr_t)s; /* non-zero default, as the reference */
    s->probs = (float*)malloc((size_t)vocab_size * sizeof(float));
    s->sorted = (float*)malloc((size_t)vocab_size * sizeof(float));
    if (!s->probs || !s->sorted) {
        bm_destroy_sampler(s);
        return NULL;
    }
    return s;
}

extern "C" void bm_destroy_sampler(bm_sampler_t* s) {
    if (!s) return;
    free(s->probs);
    free(s->sorted);
    free(s);
}

static int argmax_first(const float* v, int n) {
    int best = 0;
    for (int i = 1; i < n; i++)
        if (v[i] > v[best]) best = i;
    return best;
}

/* qsort order of floats, largest first (no shared state: samplers on
 * several threads sort at once) */
static int cmp_desc(const void* a, const void* b) {
    const float fa = *(const float*)a, fb = *(const float*)b;
    return fa > fb ? -1 : (fa < fb ? 1 : 0);
}

/* The hashed LCG step of both samplers. */
static unsigned int lcg_hash(unsigned int state) {
    unsigned int r = state * 1664525u + 1013904223u;
    r ^= r >> 13;
    r *= 1274126177u;
    r ^= r >> 16;
    return r;
}

/* temperature -> softmax -> top-k mask -> top-p mask -> inverse-CDF draw
 * with the hash value r; `fallback` when the cumulative sum never reaches
 * the target (a NaN logit).  The threshold and the cut depend on the
 * sorted values only, so a sorted copy of the values (in `sorted`, n
 * floats of the caller's) stands for the reference's sorted (value, index)
 * pairs, ties included. */
static int sample_probs(float* p, float* sorted, int n, float temperature, int top_k, float top_p, unsigned int r,
                        int fallback, const float* logits) {
    if (temperature <= 0.0f) return argmax_first(logits, n);
    for (int i = 0; i < n; i++) p[i] = logits[i] / temperature;
    float mx = -INFINITY;
    for (int i = 0; i < n; i++)
        if (p[i] > mx) mx = p[i];
    float sum = 0.0f;
    for (int i = 0; i < n; i++) {
        p[i] = expf(p[i] - mx);
        sum += p[i];
    }
    for (int i = 0; i < n; i++) p[i] /= sum;
    if (top_k > 0 && top_k < n) {
        memcpy(sorted, p, (size_t)n * sizeof(float));
        qsort(sorted, n, sizeof(float), cmp_desc);
        const float thresh = sorted[top_k - 1];
        for (int i = 0; i < n; i++)
            if (p[i] < thresh) p[i] = 0.0f;
        float s = 0.0f;
        for (int i = 0; i < n; i++) s += p[i];
        if (s > 0.0f)
            for (int i = 0; i < n; i++) p[i] /= s;
    }
    if (top_p > 0.0f && top_p < 1.0f) {
        memcpy(sorted, p, (size_t)n * sizeof(float));
        qsort(sorted, n, sizeof(float), cmp_desc);
        float cum = 0.0f, cut = 0.0f;
        for (int i = 0; i < n; i++) {
            cum += sorted[i];
            if (cum >= top_p) {
                cut = sorted[i];
                break;
            }
        }
        for (int i = 0; i < n; i++)
            if (p[i] < cut) p[i] = 0.0f;
        float s = 0.0f;
        for (int i = 0; i < n; i++) s += p[i];
        if (s > 0.0f)
            for (int i = 0; i < n; i++) p[i] /= s;
    }
    float total = 0.0f;
    for (int i = 0; i < n; i++) total += p[i];
    const float target = ((float)(r & 0xFFFFFF) / (float)0x1000000) * total;
    float c = 0.0f;
    for (int i = 0; i < n; i++) {
        c += p[i];
        if (c >= target) return i;
    }
    return fallback;
}

extern "C" int bm_sample(bm_sampler_t* s, const float* logits) {
    if (!s || !logits) return 0;
    if (s->temperature <= 0.0f) return argmax_first(logits, s->vocab_size);
    const unsigned int r = lcg_hash(s->rng);
    s->rng = r;
    return sample_probs(s->probs, s->sorted, s->vocab_size, s->temperature, s->top_k, s->topp, r, s->vocab_size - 1,
                        logits);
}

/* ------------------------------------------------------------------ */
/* driver: reference tools/run.c:121-185 */

extern "C" int bm_run_tokens(bm_context_t* ctx, bm_model_t* m, const int* prompt_ids, int n_prompt, int steps,
                             float temperature, int top_k, float top_p, uint64_t seed, bm_token_cb_t callback,
                             void* user_data) {
    if (!ctx || !m || n_prompt <= 0 || !prompt_ids) return -1;
    bm_compile(m);
    bm_session_t* S = bm_create_session(ctx, m);
    if (!S) return -1;
    int rc = 0;
    if (temperature <= 0.0f && steps >= n_prompt && steps <= S->MS) {
        /* greedy: the whole loop runs on the device, then the callback sees the tokens in order */
        int* toks = (int*)malloc((size_t)(steps - n_prompt + 1) * sizeof(int));
        const int n = toks ? bm_generate_greedy(S, prompt_ids, n_prompt, steps, toks) : -1;
        if (n < 0) rc = -1;
        for (int i = 0; i < n; i++)
            if (callback && callback(toks[i], user_data)) break;
        free(toks);
    } else {
        if (seed == 0) seed = (uint64_t)time(NULL); /* as the reference driver, run.c:135 */
        unsigned int rng_state = (unsigned int)seed;
        float* p = (float*)malloc((size_t)m->V * sizeof(float));
        float* sorted = (float*)malloc((size_t)m->V * sizeof(float));
        int next = -1;
        for (int pos = 0; pos < steps && p && sorted; pos++) {
            const int tok = pos < n_prompt ? prompt_ids[pos] : next;
            float* logits = bm_step(S, tok);
            if (!logits) {
                rc = -1;
                break;
            }
            if (pos >= n_prompt - 1) {
                next = sample_probs(p, sorted, m->V, temperature, top_k, top_p, lcg_hash(rng_state++), 0, logits);
                if (callback && callback(next, user_data)) break;
            }
        }
        if (!p || !sorted) rc = -1;
        free(p);
        free(sorted);
    }
    bm_destroy_session(S);
    return rc;
}
