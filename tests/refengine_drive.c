/* SPDX-License-Identifier: MPL-2.0
 *
 * refengine_drive.c — test driver for the reference's own C engine linked
 * against libbaremetal_hip.so in place of the Metal backend.
 *
 * Built by oracle/Makefile (`refengine`) from the reference's engine sources
 * where they lie (the inference objects of the reference Makefile's C_SRCS)
 * plus this file; the output, oracle/_ref/refengine, is test infrastructure.
 * It calls the reference's public API in the order its CLI does
 * (reference tools/cli.c:878-895: bm_load_weights, model->quant_bits,
 * model->precision, max_seq_len clamp; tools/run.c:121-185 for the greedy
 * loop), so every GPU operation it causes goes through the 22 backend.h
 * functions and the kernels the reference's scheduler resolves by name.
 *
 * usage: refengine <model_dir> <mode> <precision> <quant> <max_seq> <out> <tok>...
 *   mode "step":    bm_step over the tokens, the logits of every step to <out>
 *                   (n x vocab fp32);
 *   mode "forward": bm_forward over the tokens (prefill at position 0), then
 *                   the last position's logits to <out> (vocab fp32);
 *   mode "greedy":  bm_run_tokens with temperature 0 for <steps> = the first
 *                   token argument, the prompt = the remaining tokens; the
 *                   generated ids to <out> (int32).
 *   precision: fp32 | bf16 | fp16; quant: 8 | 4 | 0.
 * Exit status 0 on success; 2 on a usage error; 3 if the engine failed.
 */
#include "baremetal.h"
#include "baremetal/model.h"

#include <stdio.h>
#include <stdlib.h>
#include <string.h>

typedef struct {
    int* ids;
    int n, cap;
} collect_t;

static int collect(int token_id, void* ud) {
    collect_t* c = (collect_t*)ud;
    if (c->n == c->cap) {
        c->cap = c->cap ? 2 * c->cap : 64;
        int* p = (int*)realloc(c->ids, (size_t)c->cap * sizeof(int));
        if (!p) return 1;
        c->ids = p;
    }
    c->ids[c->n++] = token_id;
    return 0;
}

int main(int argc, char** argv) {
    if (argc < 8) {
        fprintf(stderr, "usage: %s <model_dir> <step|forward|greedy> <fp32|bf16> <quant> <max_seq> <out> <tok>...\n",
                argv[0]);
        return 2;
    }
    const char* dir = argv[1];
    const char* mode = argv[2];
    const char* prec = argv[3];
    const int quant = atoi(argv[4]);
    const int max_seq = atoi(argv[5]);
    const char* out = argv[6];
    const int n = argc - 7;
    int* toks = (int*)malloc((size_t)n * sizeof(int));
    if (!toks) return 3;
    for (int i = 0; i < n; i++) toks[i] = atoi(argv[7 + i]);

    bm_context_t* ctx = bm_create(BM_DEVICE_METAL);
    if (!ctx) return 3;
    bm_model_t* model = (bm_model_t*)calloc(1, sizeof(*model));
    bm_load_weights(model, dir);
    if (!model->weight_buffer) {
        fprintf(stderr, "refengine: failed to load weights from %s\n", dir);
        return 3;
    }
    model->quant_bits = quant;
    model->precision = strcmp(prec, "bf16") == 0   ? BM_PRECISION_BF16
                       : strcmp(prec, "fp16") == 0 ? BM_PRECISION_FP16
                                                   : BM_PRECISION_FP32;
    if (max_seq > 0 && model->arch.max_seq_len > max_seq) model->arch.max_seq_len = max_seq;
    const int V = model->arch.vocab_size;

    FILE* f = fopen(out, "wb");
    if (!f) return 3;
    int rc = 0;
    if (strcmp(mode, "greedy") == 0) {
        if (n < 2) return 2;
        collect_t c = {NULL, 0, 0};
        rc = bm_run_tokens(ctx, model, toks + 1, n - 1, toks[0], 0.0f, 0, 1.0f, 1, collect, &c);
        if (rc == 0 && c.n > 0 && fwrite(c.ids, sizeof(int), (size_t)c.n, f) != (size_t)c.n) rc = 3;
        free(c.ids);
    } else {
        bm_compile(model);
        bm_session_t* s = bm_create_session(ctx, model);
        if (!s) {
            rc = 3;
        } else if (strcmp(mode, "forward") == 0) {
            const float* lg = bm_forward(s, toks, n);
            if (!lg || fwrite(lg, sizeof(float), (size_t)V, f) != (size_t)V) rc = 3;
        } else {
            for (int i = 0; i < n && rc == 0; i++) {
                const float* lg = bm_step(s, toks[i]);
                if (!lg || fwrite(lg, sizeof(float), (size_t)V, f) != (size_t)V) rc = 3;
            }
        }
        if (s) bm_destroy_session(s);
    }
    fclose(f);
    bm_destroy_model(model);
    bm_destroy(ctx);
    free(toks);
    return rc ? 3 : 0;
}
