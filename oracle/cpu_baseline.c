/* SPDX-License-Identifier: MPL-2.0
 *
 * cpu_baseline.c — the host-CPU Q8 matvec that bench.py times beside the GPU
 * (TEST/BENCH INFRASTRUCTURE ONLY; never linked into the product).
 *
 * The reference has no CPU compute path (its CPU context creates no backend,
 * reference src/baremetal/context.c:16-22), so the baseline is this C
 * restatement of the reference's Q8 matvec arithmetic (reference
 * src/kernels/forward.metal:575-623: per block, dot of 32 int8 weights with
 * 32 fp32 activations, times the block scale, summed over blocks), written
 * for the host, rows split over OpenMP threads.  On AVX-512 (BW) hosts an
 * explicit loop: a block's 32 int8 codes sign-extended to two 16-lane int32
 * vectors (vpmovsxbd), converted to fp32 and multiplied into the 32
 * activations (two FMAs), the block product scaled into a 16-lane
 * accumulator, one horizontal sum per row.  Elsewhere the portable loop:
 * 16 independent fp32 partial sums per block so the compiler vectorises it
 * (AVX2 / baseline x86-64 picked at load time by target_clones).
 */
#include "oracle.h"

#include <immintrin.h>
#include <omp.h>
#include <string.h>

__attribute__((target("avx512f,avx512bw,avx512vl")))
static void rows_avx512(const uint8_t* w, const float* x, float* y, int C, int r0, int r1) {
    const int nb = C / 32;
    for (int r = r0; r < r1; r++) {
        const uint8_t* row = w + (size_t)r * nb * 36;
        __m512 acc = _mm512_setzero_ps();
        for (int b = 0; b < nb; b++) {
            const uint8_t* blk = row + (size_t)b * 36;
            float s;
            memcpy(&s, blk, 4);
            const __m256i q = _mm256_loadu_si256((const __m256i*)(blk + 4));
            const __m512 q0 = _mm512_cvtepi32_ps(_mm512_cvtepi8_epi32(_mm256_castsi256_si128(q)));
            const __m512 q1 = _mm512_cvtepi32_ps(_mm512_cvtepi8_epi32(_mm256_extracti128_si256(q, 1)));
            __m512 p = _mm512_mul_ps(q0, _mm512_loadu_ps(x + 32 * b));
            p = _mm512_fmadd_ps(q1, _mm512_loadu_ps(x + 32 * b + 16), p);
            acc = _mm512_fmadd_ps(_mm512_set1_ps(s), p, acc);
        }
        y[r] = _mm512_reduce_add_ps(acc);
    }
}

__attribute__((target_clones("avx2", "default")))
static void rows_portable(const uint8_t* w, const float* x, float* y, int C, int r0, int r1) {
    const int nb = C / 32;
    for (int r = r0; r < r1; r++) {
        const uint8_t* row = w + (size_t)r * nb * 36;
        float acc = 0.0f;
        for (int b = 0; b < nb; b++) {
            const uint8_t* blk = row + (size_t)b * 36;
            float s;
            memcpy(&s, blk, 4);
            const int8_t* q = (const int8_t*)(blk + 4);
            const float* xb = x + 32 * b;
            float p[16] = {0};
            for (int j = 0; j < 32; j++) p[j & 15] += xb[j] * (float)q[j];
            float part = 0.0f;
            for (int j = 0; j < 16; j++) part += p[j];
            acc += part * s;
        }
        y[r] = acc;
    }
}

static int has_avx512bw(void) {
    __builtin_cpu_init();
    return __builtin_cpu_supports("avx512f") && __builtin_cpu_supports("avx512bw") && __builtin_cpu_supports("avx512vl");
}

static void rows_f32(const uint8_t* w, const float* x, float* y, int C, int r0, int r1) {
    if (has_avx512bw()) rows_avx512(w, x, y, C, r0, r1);
    else rows_portable(w, x, y, C, r0, r1);
}

void orc_cpu_q8_matvec_f32(const uint8_t* w, const float* x, float* y, int C, int OC, int nthreads) {
    if (nthreads < 1) nthreads = 1;
#pragma omp parallel num_threads(nthreads)
    {
        int t = omp_get_thread_num(), nt = omp_get_num_threads();
        int r0 = (int)((long)OC * t / nt), r1 = (int)((long)OC * (t + 1) / nt);
        rows_f32(w, x, y, C, r0, r1);
    }
}

/* Many independent problems (one decode token's projections): the rows of
 * all problems form one index space split evenly over the threads. */
void orc_cpu_q8_matvec_multi(const uint8_t* w, const float* x, float* y, int nprob, const uint64_t* w_off,
                             const uint64_t* x_off, const uint64_t* y_off, const int* OC, const int* C,
                             int nthreads) {
    if (nthreads < 1) nthreads = 1;
    long total = 0;
    for (int i = 0; i < nprob; i++) total += OC[i];
#pragma omp parallel num_threads(nthreads)
    {
        int t = omp_get_thread_num(), nt = omp_get_num_threads();
        long g0 = total * t / nt, g1 = total * (t + 1) / nt, base = 0;
        for (int i = 0; i < nprob && base < g1; i++) {
            long r0 = g0 > base ? g0 - base : 0, r1 = g1 - base < OC[i] ? g1 - base : OC[i];
            if (r0 < r1)
                rows_f32(w + w_off[i], x + x_off[i], y + y_off[i], C[i], (int)r0, (int)r1);
            base += OC[i];
        }
    }
}

int orc_cpu_max_threads(void) { return omp_get_max_threads(); }

const char* orc_cpu_isa(void) {
    __builtin_cpu_init();
    if (has_avx512bw()) return "avx512bw (explicit int8 widen + fma)";
    if (__builtin_cpu_supports("avx2")) return "avx2 (auto-vectorised)";
    return "x86-64";
}

/* ---- fp32 SIMD decode step (the config-5 CPU baseline) ----------------
 * The reference's decode graph (src/baremetal/graph.c:126-226) on the host
 * in fp32, as the GPU computes it: RMSNorm (forward.metal:1019-1060),
 * q/k/v Q8 matvecs (:575-623), rotate-half RoPE (:1260-1313), KV store and
 * GQA attention with scale 1/sqrt(HD) over S = pos + 1 keys (:1317-1465),
 * o matvec + residual, RMSNorm, gate/up, SiLU gate (:1179-1190), down +
 * residual, final RMSNorm and the fp32 tied LM head (:1636-1689).  Every
 * matvec is split over the threads by rows and vectorised like rows_f32;
 * the other ops are serial (they are a small part of a token).  This is a
 * timing baseline; the fp64 decoder in decode_oracle.c is the checker. */
#include "decode_oracle.h"

#include <math.h>
#include <stdlib.h>

typedef struct {
    orc_model_t m;
    float *kv, *x, *xn, *q, *k, *v, *att, *o, *g, *u, *dn, *sc, *logits;
    int nt;
} cpu_dec_t;

__attribute__((target_clones("avx512f", "avx2", "default")))
static void head_rows(const float* w, const float* x, float* y, int C, int r0, int r1) {
    for (int r = r0; r < r1; r++) {
        const float* row = w + (size_t)r * C;
        float p[16] = {0};
        for (int j = 0; j < C; j++) p[j & 15] += row[j] * x[j];
        float acc = 0.0f;
        for (int j = 0; j < 16; j++) acc += p[j];
        y[r] = acc;
    }
}

static void cpu_mv(const uint8_t* w, const float* x, float* y, int C, int OC, int nt) {
#pragma omp parallel num_threads(nt)
    {
        int t = omp_get_thread_num(), n = omp_get_num_threads();
        rows_f32(w, x, y, C, (int)((long)OC * t / n), (int)((long)OC * (t + 1) / n));
    }
}

static void cpu_rmsnorm(const float* x, const float* w, float* out, int C, float eps) {
    float ss = 0.0f;
    for (int j = 0; j < C; j++) ss += x[j] * x[j];
    const float inv = 1.0f / sqrtf(ss / (float)C + eps);
    for (int j = 0; j < C; j++) out[j] = (x[j] * inv) * w[j];
}

void* orc_cpu_decoder_create(const void* mp, int nthreads) {
    const orc_model_t* m = (const orc_model_t*)mp;
    if (m->qbits == 4 || m->head_q8) return NULL; /* Q8 projections + fp32 head only */
    cpu_dec_t* d = (cpu_dec_t*)calloc(1, sizeof(cpu_dec_t));
    if (!d) return NULL;
    d->m = *m;
    d->nt = nthreads > 0 ? nthreads : 1;
    const int KV = m->NKV * m->HD, QD = m->NH * m->HD;
    d->kv = (float*)calloc((size_t)m->L * 2 * m->MS * KV, sizeof(float));
    d->x = (float*)calloc(m->D, 4);
    d->xn = (float*)calloc(m->H > m->D ? m->H : m->D, 4);
    d->q = (float*)calloc(QD, 4);
    d->k = (float*)calloc(KV, 4);
    d->v = (float*)calloc(KV, 4);
    d->att = (float*)calloc(QD, 4);
    d->o = (float*)calloc(m->D, 4);
    d->g = (float*)calloc(m->H, 4);
    d->u = (float*)calloc(m->H, 4);
    d->dn = (float*)calloc(m->D, 4);
    d->sc = (float*)calloc(m->MS, 4);
    d->logits = (float*)calloc(m->V, 4);
    if (!d->kv || !d->x || !d->xn || !d->q || !d->k || !d->v || !d->att || !d->o || !d->g || !d->u || !d->dn ||
        !d->sc || !d->logits) {
        orc_cpu_decoder_destroy(d);
        return NULL;
    }
    return d;
}

void orc_cpu_decoder_destroy(void* p) {
    cpu_dec_t* d = (cpu_dec_t*)p;
    if (!d) return;
    free(d->kv); free(d->x); free(d->xn); free(d->q); free(d->k); free(d->v); free(d->att);
    free(d->o); free(d->g); free(d->u); free(d->dn); free(d->sc); free(d->logits);
    free(d);
}

/* One token at position pos; returns the greedy pick (first maximum) or -1. */
int orc_cpu_decoder_step(void* p, int token, int pos, float* logits_out) {
    cpu_dec_t* d = (cpu_dec_t*)p;
    const orc_model_t* m = &d->m;
    const int D = m->D, H = m->H, NH = m->NH, NKV = m->NKV, HD = m->HD, V = m->V, MS = m->MS;
    const int KV = NKV * HD, QD = NH * HD, kv_mul = NH / NKV, nt = d->nt;
    const size_t bD = (size_t)(D / 32) * 36, bH = (size_t)(H / 32) * 36, bQ = (size_t)(QD / 32) * 36;
    if (token < 0 || token >= V || pos < 0 || pos >= MS) return -1;
    memcpy(d->x, m->emb + (size_t)token * D, (size_t)D * 4);
    const float scale = 1.0f / sqrtf((float)HD);
    for (int l = 0; l < m->L; l++) {
        cpu_rmsnorm(d->x, m->ln1 + (size_t)l * D, d->xn, D, m->eps);
        cpu_mv(m->wq + (size_t)l * QD * bD, d->xn, d->q, D, QD, nt);
        cpu_mv(m->wk + (size_t)l * KV * bD, d->xn, d->k, D, KV, nt);
        cpu_mv(m->wv + (size_t)l * KV * bD, d->xn, d->v, D, KV, nt);
        for (int i = 0; i < HD / 2; i++) {
            const float ang = (float)pos * (1.0f / powf(m->theta, (float)(2 * i) / (float)HD));
            const float c = cosf(ang), s = sinf(ang);
            for (int h = 0; h < NH; h++) {
                float* qh = d->q + h * HD;
                const float a0 = qh[i], a1 = qh[i + HD / 2];
                qh[i] = a0 * c - a1 * s;
                qh[i + HD / 2] = a0 * s + a1 * c;
            }
            for (int h = 0; h < NKV; h++) {
                float* kh = d->k + h * HD;
                const float b0 = kh[i], b1 = kh[i + HD / 2];
                kh[i] = b0 * c - b1 * s;
                kh[i + HD / 2] = b0 * s + b1 * c;
            }
        }
        float* kc = d->kv + (size_t)l * 2 * MS * KV;
        float* vc = kc + (size_t)MS * KV;
        memcpy(kc + (size_t)pos * KV, d->k, (size_t)KV * 4);
        memcpy(vc + (size_t)pos * KV, d->v, (size_t)KV * 4);
        const int S = pos + 1;
        for (int h = 0; h < NH; h++) {
            const int kh = h / kv_mul;
            const float* qh = d->q + h * HD;
            float mx = -INFINITY;
            for (int t = 0; t < S; t++) {
                const float* kr = kc + (size_t)t * KV + kh * HD;
                float sd = 0.0f;
                for (int i = 0; i < HD; i++) sd += qh[i] * kr[i];
                d->sc[t] = sd * scale;
                mx = d->sc[t] > mx ? d->sc[t] : mx;
            }
            float den = 0.0f;
            for (int t = 0; t < S; t++) {
                d->sc[t] = expf(d->sc[t] - mx);
                den += d->sc[t];
            }
            float* ah = d->att + h * HD;
            for (int i = 0; i < HD; i++) ah[i] = 0.0f;
            for (int t = 0; t < S; t++) {
                const float* vr = vc + (size_t)t * KV + kh * HD;
                const float wgt = d->sc[t] / den;
                for (int i = 0; i < HD; i++) ah[i] += wgt * vr[i];
            }
        }
        cpu_mv(m->wo + (size_t)l * D * bQ, d->att, d->o, QD, D, nt);
        for (int j = 0; j < D; j++) d->x[j] += d->o[j];
        cpu_rmsnorm(d->x, m->ln2 + (size_t)l * D, d->xn, D, m->eps);
        cpu_mv(m->wg + (size_t)l * H * bD, d->xn, d->g, D, H, nt);
        cpu_mv(m->wu + (size_t)l * H * bD, d->xn, d->u, D, H, nt);
        for (int j = 0; j < H; j++) d->g[j] = d->g[j] / (1.0f + expf(-d->g[j])) * d->u[j];
        cpu_mv(m->wd + (size_t)l * D * bH, d->g, d->dn, H, D, nt);
        for (int j = 0; j < D; j++) d->x[j] += d->dn[j];
    }
    cpu_rmsnorm(d->x, m->lnf, d->xn, D, m->eps);
    const float* hw = m->head_f32 ? m->head_f32 : m->emb;
#pragma omp parallel num_threads(nt)
    {
        int t = omp_get_thread_num(), n = omp_get_num_threads();
        head_rows(hw, d->xn, d->logits, D, (int)((long)V * t / n), (int)((long)V * (t + 1) / n));
    }
    int best = 0;
    for (int i = 1; i < V; i++)
        if (d->logits[i] > d->logits[best]) best = i;
    if (logits_out) memcpy(logits_out, d->logits, (size_t)V * 4);
    return best;
}
