/* SPDX-License-Identifier: MPL-2.0
 *
 * decode_oracle.h — CPU restatement of the reference's decode step (test
 * infrastructure only; see decode_oracle.c).
 */
#ifndef BM_DECODE_ORACLE_H
#define BM_DECODE_ORACLE_H

#include <stdint.h>

/* Weights as the reference lays them out (model.c:125-172): per matrix
 * type, all layers back to back; quantized matrices as rows of C/32 blocks
 * (Q8_0 36 bytes, Q4_0 20 bytes). */
typedef struct {
    int D, H, NH, NKV, HD, L, V, MS;
    float theta, eps;
    const float* emb;        /* [V][D] fp32, also the tied LM head */
    const float* ln1;        /* [L][D] */
    const float* ln2;        /* [L][D] */
    const float* lnf;        /* [D] */
    const uint8_t* wq;       /* [L][NH*HD][D/32] */
    const uint8_t* wk;       /* [L][KV][D/32] */
    const uint8_t* wv;       /* [L][KV][D/32] */
    const uint8_t* wo;       /* [L][D][NH*HD/32] */
    const uint8_t* wg;       /* [L][H][D/32] */
    const uint8_t* wu;       /* [L][H][D/32] */
    const uint8_t* wd;       /* [L][D][H/32] */
    const uint8_t* head_q8;  /* NULL: fp32 tied head (the reference's Q8 mode) */
    const float* head_f32;   /* fp32 head rows [V][D] when head_q8 is NULL; NULL: emb.  The
                                reference's bf16 head is emb rounded to bf16 and widened back */
    int qbits;               /* projections: 8 (or 0) Q8_0 36-byte blocks, 4 Q4_0 20-byte blocks */
} orc_model_t;

typedef struct orc_decoder_s orc_decoder_t;

orc_decoder_t* orc_decoder_create(const orc_model_t* m, int nthreads);
void orc_decoder_destroy(orc_decoder_t* d);
/* One token at position pos; writes V logits.  Returns 0 or -1. */
int orc_decoder_step(orc_decoder_t* d, int token, int pos, double* logits);
int orc_argmax_first(const double* v, int n, double* top1, double* top2);
/* Rotate-half RoPE in place (the step's own), and the last layer's attention
 * output of the last step (NH*HD floats). */
void orc_rope(float* v, int nheads, int HD, int pos, float theta);
void orc_decoder_last_attention(const orc_decoder_t* d, float* out);
/* Greedy run in the reference's driver order (tools/run.c:121-185): step
 * prompt tokens, then the previous pick (or forced[] when non-NULL, for
 * teacher forcing).  Emits steps-n_prompt+1 tokens and their top-2 margins;
 * returns the count or -1. */
int orc_generate(orc_decoder_t* d, const int* prompt, int n_prompt, int steps, const int* forced, int* out_tokens,
                 double* out_margin);

#endif
