/* SPDX-License-Identifier: MPL-2.0
 *
 * decode_oracle.c — CPU restatement of the reference's single-token decode
 * step with Q8 projections (TEST INFRASTRUCTURE ONLY, see oracle.c).
 *
 * Op order follows the reference's decode graph (src/baremetal/graph.c:126-226):
 * per layer  rmsnorm -> q,k,v (Q8) -> rope -> kv_store + attention -> o (Q8)
 *            -> residual add -> rmsnorm -> gate,up (Q8) -> swiglu -> down (Q8)
 *            -> residual add;
 * then the fused final rmsnorm + LM head (src/baremetal/compiler.c:67-110,
 * forward.metal:1636-1689) over the tied fp32 embedding (model.c:168-169),
 * or, as an extension, a Q8 LM head; then first-max argmax
 * (tools/run.c:56-60, sampler.c:36-40).
 * Elementwise formulas: rmsnorm (forward.metal:1019-1060, eps 1e-5 from
 * graph.c:134), rope_inv_freq + rope_forward (forward.metal:1260-1313),
 * kv_store (:1317-1329), attention_forward (:1362-1465, scale 1/sqrt(HD)
 * from scheduler.c:914, S = pos+1 from scheduler.c:808), swiglu
 * (:1179-1190), add (:1332-1340).
 *
 * Precision: every buffer the reference keeps in fp32 is kept in fp32 here
 * (activations, KV cache, the rope angle pos*freq), and every reduction
 * (dot products, sums of squares, softmax sums) is carried in double, so
 * the result is the reference's arithmetic without its summation-order
 * noise.
 */
#include "decode_oracle.h"
#include "oracle.h"

#include <math.h>
#include <omp.h>
#include <stdlib.h>
#include <string.h>

struct orc_decoder_s {
    orc_model_t m;
    float* kv;     /* [L][2][MS][KV] */
    float* x;      /* [D] residual */
    float* xn;     /* [D] */
    float* q;      /* [NH*HD] */
    float* k;      /* [KV] */
    float* v;      /* [KV] */
    float* att;    /* [NH*HD] */
    float* o;      /* [D] */
    float* g;      /* [H] */
    float* u;      /* [H] */
    float* dn;     /* [D] */
    double* sc;    /* [MS] scores */
    int nthreads;
};

static void rmsnorm(const float* x, const float* w, float* out, int C, float eps) {
    double ss = 0.0;
    for (int j = 0; j < C; j++) ss += (double)x[j] * (double)x[j];
    float msf = (float)ss / (float)C;
    float inv = 1.0f / sqrtf(msf + eps);
    for (int j = 0; j < C; j++) out[j] = (x[j] * inv) * w[j];
}

static void q8_mv(const uint8_t* w, const float* x, float* y, int C, int OC, int nt) {
    const int nb = C / 32;
#pragma omp parallel for num_threads(nt) schedule(static)
    for (int r = 0; r < OC; r++) {
        const uint8_t* row = w + (size_t)r * nb * 36;
        double acc = 0.0;
        for (int b = 0; b < nb; b++) {
            float s;
            memcpy(&s, row + (size_t)b * 36, 4);
            const int8_t* q = (const int8_t*)(row + (size_t)b * 36 + 4);
            double part = 0.0;
            for (int j = 0; j < 32; j++) part += (double)x[32 * b + j] * (double)q[j];
            acc += (double)s * part;
        }
        y[r] = (float)acc;
    }
}

/* Q4_0 rows (reference forward.metal:654-858): 20-byte blocks, element 2j
 * in the low nibble of byte j, 2j+1 in the high nibble, codes in [-8, 7]. */
static void q4_mv(const uint8_t* w, const float* x, float* y, int C, int OC, int nt) {
    const int nb = C / 32;
#pragma omp parallel for num_threads(nt) schedule(static)
    for (int r = 0; r < OC; r++) {
        const uint8_t* row = w + (size_t)r * nb * 20;
        double acc = 0.0;
        for (int b = 0; b < nb; b++) {
            float s;
            memcpy(&s, row + (size_t)b * 20, 4);
            const uint8_t* qs = row + (size_t)b * 20 + 4;
            double part = 0.0;
            for (int j = 0; j < 32; j++) {
                const int nib = (qs[j >> 1] >> (4 * (j & 1))) & 0x0F;
                part += (double)x[32 * b + j] * (double)(nib >= 8 ? nib - 16 : nib);
            }
            acc += (double)s * part;
        }
        y[r] = (float)acc;
    }
}

/* the model's projection format */
static void proj_mv(const orc_model_t* m, const uint8_t* w, const float* x, float* y, int C, int OC, int nt) {
    if (m->qbits == 4) q4_mv(w, x, y, C, OC, nt);
    else q8_mv(w, x, y, C, OC, nt);
}

static void f32_mv(const float* w, const float* x, double* y, int C, int OC, int nt) {
#pragma omp parallel for num_threads(nt) schedule(static)
    for (int r = 0; r < OC; r++) {
        const float* row = w + (size_t)r * C;
        double acc = 0.0;
        for (int j = 0; j < C; j++) acc += (double)row[j] * (double)x[j];
        y[r] = acc;
    }
}

static float rope_freq(float theta, int i, int HD) {
    return 1.0f / powf(theta, (float)(2 * i) / (float)HD);
}

/* Rotate-half RoPE of nheads heads of HD floats at position pos (reference
 * forward.metal:1260-1263 frequencies, :1302-1310 rotation): element i of a
 * head pairs with element i + HD/2, angle pos * theta^(-2i/HD) taken in
 * fp32, cos/sin of that angle. */
void orc_rope(float* v, int nheads, int HD, int pos, float theta) {
    for (int i = 0; i < HD / 2; i++) {
        float fr = rope_freq(theta, i, HD);
        float ang = (float)pos * fr;
        float c = (float)cos((double)ang), s = (float)sin((double)ang);
        for (int h = 0; h < nheads; h++) {
            float* vh = v + h * HD;
            float a0 = vh[i], a1 = vh[i + HD / 2];
            vh[i] = a0 * c - a1 * s;
            vh[i + HD / 2] = a0 * s + a1 * c;
        }
    }
}

orc_decoder_t* orc_decoder_create(const orc_model_t* m, int nthreads) {
    orc_decoder_t* d = (orc_decoder_t*)calloc(1, sizeof(orc_decoder_t));
    if (!d) return NULL;
    d->m = *m;
    const int KV = m->NKV * m->HD, QD = m->NH * m->HD;
    d->kv = (float*)calloc((size_t)m->L * 2 * m->MS * KV, sizeof(float));
    d->x = (float*)calloc(m->D, sizeof(float));
    d->xn = (float*)calloc(m->D, sizeof(float));
    d->q = (float*)calloc(QD, sizeof(float));
    d->k = (float*)calloc(KV, sizeof(float));
    d->v = (float*)calloc(KV, sizeof(float));
    d->att = (float*)calloc(QD, sizeof(float));
    d->o = (float*)calloc(m->D, sizeof(float));
    d->g = (float*)calloc(m->H, sizeof(float));
    d->u = (float*)calloc(m->H, sizeof(float));
    d->dn = (float*)calloc(m->D, sizeof(float));
    d->sc = (double*)calloc(m->MS, sizeof(double));
    d->nthreads = nthreads > 0 ? nthreads : 1;
    if (!d->kv || !d->x || !d->xn || !d->q || !d->k || !d->v || !d->att || !d->o || !d->g || !d->u || !d->dn ||
        !d->sc) {
        orc_decoder_destroy(d);
        return NULL;
    }
    return d;
}

void orc_decoder_destroy(orc_decoder_t* d) {
    if (!d) return;
    free(d->kv); free(d->x); free(d->xn); free(d->q); free(d->k); free(d->v);
    free(d->att); free(d->o); free(d->g); free(d->u); free(d->dn); free(d->sc);
    free(d);
}

int orc_decoder_step(orc_decoder_t* d, int token, int pos, double* logits) {
    const orc_model_t* m = &d->m;
    const int D = m->D, H = m->H, NH = m->NH, NKV = m->NKV, HD = m->HD, L = m->L, V = m->V, MS = m->MS;
    const int KV = NKV * HD, QD = NH * HD, nbD = D / 32, nbH = H / 32, nbQ = QD / 32;
    const size_t bb = m->qbits == 4 ? 20 : 36; /* bytes per projection block */
    const int kv_mul = NH / NKV, nt = d->nthreads;
    if (token < 0 || token >= V || pos < 0 || pos >= MS) return -1;

    memcpy(d->x, m->emb + (size_t)token * D, (size_t)D * sizeof(float));
    const float scale = 1.0f / sqrtf((float)HD);

    for (int l = 0; l < L; l++) {
        rmsnorm(d->x, m->ln1 + (size_t)l * D, d->xn, D, m->eps);
        proj_mv(m, m->wq + (size_t)l * QD * nbD * bb, d->xn, d->q, D, QD, nt);
        proj_mv(m, m->wk + (size_t)l * KV * nbD * bb, d->xn, d->k, D, KV, nt);
        proj_mv(m, m->wv + (size_t)l * KV * nbD * bb, d->xn, d->v, D, KV, nt);

        orc_rope(d->q, NH, HD, pos, m->theta);
        orc_rope(d->k, NKV, HD, pos, m->theta);

        float* kc = d->kv + (size_t)l * 2 * MS * KV;
        float* vc = kc + (size_t)MS * KV;
        memcpy(kc + (size_t)pos * KV, d->k, (size_t)KV * sizeof(float));
        memcpy(vc + (size_t)pos * KV, d->v, (size_t)KV * sizeof(float));

        const int S = pos + 1;
        for (int h = 0; h < NH; h++) {
            const int kh = h / kv_mul;
            const float* qh = d->q + h * HD;
            double mx = -INFINITY;
            for (int t = 0; t < S; t++) {
                const float* kr = kc + (size_t)t * KV + kh * HD;
                double sdot = 0.0;
                for (int i = 0; i < HD; i++) sdot += (double)qh[i] * (double)kr[i];
                d->sc[t] = sdot * (double)scale;
                if (d->sc[t] > mx) mx = d->sc[t];
            }
            double den = 0.0;
            for (int t = 0; t < S; t++) {
                d->sc[t] = exp(d->sc[t] - mx);
                den += d->sc[t];
            }
            for (int i = 0; i < HD; i++) {
                double acc = 0.0;
                for (int t = 0; t < S; t++) acc += d->sc[t] * (double)vc[(size_t)t * KV + kh * HD + i];
                d->att[h * HD + i] = (float)(acc / den);
            }
        }

        proj_mv(m, m->wo + (size_t)l * D * nbQ * bb, d->att, d->o, QD, D, nt);
        for (int j = 0; j < D; j++) d->x[j] = d->x[j] + d->o[j];

        rmsnorm(d->x, m->ln2 + (size_t)l * D, d->xn, D, m->eps);
        proj_mv(m, m->wg + (size_t)l * H * nbD * bb, d->xn, d->g, D, H, nt);
        proj_mv(m, m->wu + (size_t)l * H * nbD * bb, d->xn, d->u, D, H, nt);
        for (int j = 0; j < H; j++) {
            float gx = d->g[j];
            float silu = gx / (1.0f + expf(-gx));
            d->g[j] = silu * d->u[j];
        }
        proj_mv(m, m->wd + (size_t)l * D * nbH * bb, d->g, d->dn, H, D, nt);
        for (int j = 0; j < D; j++) d->x[j] = d->x[j] + d->dn[j];
    }

    rmsnorm(d->x, m->lnf, d->xn, D, m->eps);
    if (m->head_q8) {
        float* tmp = (float*)malloc((size_t)V * sizeof(float));
        if (!tmp) return -1;
        q8_mv(m->head_q8, d->xn, tmp, D, V, nt);
        for (int r = 0; r < V; r++) logits[r] = (double)tmp[r];
        free(tmp);
    } else {
        f32_mv(m->head_f32 ? m->head_f32 : m->emb, d->xn, logits, D, V, nt);
    }
    return 0;
}

/* The attention output (NH*HD floats, before the o projection) of the last
 * layer of the last step; for tests that look inside the step. */
void orc_decoder_last_attention(const orc_decoder_t* d, float* out) {
    memcpy(out, d->att, (size_t)d->m.NH * d->m.HD * sizeof(float));
}

int orc_argmax_first(const double* v, int n, double* top1, double* top2) {
    int best = 0;
    for (int i = 1; i < n; i++)
        if (v[i] > v[best]) best = i;
    double second = -INFINITY;
    for (int i = 0; i < n; i++)
        if (i != best && v[i] > second) second = v[i];
    if (top1) *top1 = v[best];
    if (top2) *top2 = second;
    return best;
}

int orc_generate(orc_decoder_t* d, const int* prompt, int n_prompt, int steps, const int* forced, int* out_tokens,
                 double* out_margin) {
    const int V = d->m.V;
    double* logits = (double*)malloc((size_t)V * sizeof(double));
    if (!logits) return -1;
    int next = -1, n_out = 0;
    for (int pos = 0; pos < steps; pos++) {
        int tok = pos < n_prompt ? prompt[pos] : (forced ? forced[pos - n_prompt] : next);
        if (orc_decoder_step(d, tok, pos, logits) != 0) {
            free(logits);
            return -1;
        }
        if (pos >= n_prompt - 1) {
            double t1, t2;
            next = orc_argmax_first(logits, V, &t1, &t2);
            out_tokens[n_out] = next;
            if (out_margin) out_margin[n_out] = t1 - t2;
            n_out++;
        }
    }
    free(logits);
    return n_out;
}
