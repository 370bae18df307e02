/* SPDX-License-Identifier: MPL-2.0
 *
 * baremetal.h — the engine API of the MI355X decode path.
 *
 * The types and the functions in the first part keep the names, argument
 * meanings and return conventions of the reference's public API
 * (reference include/baremetal.h:16-206), restricted to Q8 inference:
 * a context on the GPU, a model described by bm_arch_t, bm_compile, a
 * session, bm_step / bm_forward and the greedy/sampling driver
 * bm_run_tokens.  The second part holds MI355X additions that have no
 * counterpart in the reference (weight input without a checkpoint loader,
 * batched sessions, device-driven greedy generation).
 *
 * Differences a caller of the reference sees:
 *   - BM_DEVICE_METAL selects "the GPU", here the HIP device; BM_DEVICE_HIP
 *     is the same value.  BM_DEVICE_CPU has no backend, as in the reference
 *     (reference src/baremetal/context.c:16-22), and bm_create returns NULL.
 *   - Projections run in Q8_0 (quant_bits 8, the default) or Q4_0
 *     (quant_bits 4).  The LM head runs over the
 *     tied embedding in the model's precision, as the reference's Q8 mode
 *     does (reference src/baremetal/graph.c:228-238, scheduler.c:369-371,
 *     776-778): fp32 rows (BM_PRECISION_FP32) or bf16 rows rounded to
 *     nearest even (BM_PRECISION_BF16, what bm_get_supported_precision
 *     returns); or, on request, Q8 rows.  BM_PRECISION_FP16 is rejected.
 *   - Weights come from a Hugging Face checkpoint directory (bm_load_model,
 *     bm_load_weights), bm_model_set_tensor(_bf16) or
 *     bm_model_init_synthetic; the reference's own .bin checkpoint format
 *     and the tokenizer are not read.
 *   - bm_forward over several tokens at position 0 of a batch-1 session
 *     runs the whole prompt in one pass, as the reference's prefill does
 *     (reference src/baremetal/session.c:86-149); elsewhere it steps the
 *     tokens one at a time.  The logits it returns are those of the last
 *     token either way.
 */
#ifndef BAREMETAL_H
#define BAREMETAL_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- Architecture descriptor (reference include/baremetal.h:18-87) ---- */

typedef enum { BM_NORM_LAYERNORM, BM_NORM_RMSNORM } bm_norm_t;
typedef enum { BM_ACT_GELU, BM_ACT_SWIGLU } bm_act_t;
typedef enum { BM_POS_LEARNED, BM_POS_ROPE } bm_pos_t;
typedef enum { BM_ATTN_MHA, BM_ATTN_GQA } bm_attn_t;
typedef enum { BM_ROPE_NONE = 0, BM_ROPE_LLAMA3 = 1 } bm_rope_scaling_t;
typedef enum { BM_PRECISION_FP32, BM_PRECISION_FP16, BM_PRECISION_BF16 } bm_precision_t;
typedef enum { BM_DEVICE_CPU, BM_DEVICE_METAL, BM_DEVICE_HIP = BM_DEVICE_METAL } bm_device_t;

typedef struct {
    int dim;
    int hidden_dim;
    int n_layers;
    int n_heads;
    int n_kv_heads;
    int vocab_size;
    int padded_vocab_size;
    int max_seq_len;

    bm_norm_t      norm;
    bm_act_t       activation;
    bm_pos_t       pos_enc;
    bm_attn_t      attention;
    bm_precision_t precision;

    int bias;
    int weight_tie;
    int has_qk_norm;
    int has_ffn_post_norm;
    int head_dim;
    int gated_mlp;
    int gemma_norm;
    int embed_scale;
    int weight_layout;

    float rope_theta;

    bm_rope_scaling_t rope_scaling;
    float rope_factor;
    float rope_low_freq_factor;
    float rope_high_freq_factor;
    float rope_original_max;
} bm_arch_t;

typedef struct bm_context_s bm_context_t;
typedef struct bm_model_s   bm_model_t;
typedef struct bm_session_s bm_session_t;
typedef struct bm_sampler_s bm_sampler_t;

/* ---- Reference API (reference include/baremetal.h:120-175) ---- */

bm_context_t*  bm_create(bm_device_t device);
void           bm_destroy(bm_context_t* ctx);
bm_precision_t bm_get_supported_precision(bm_context_t* ctx);

/* Accepts the SmolLM2 / llama family the decode path implements: RMSNorm,
 * SwiGLU gated MLP, RoPE, GQA, tied or untied head, no biases.  NULL (logged)
 * for anything else. */
bm_model_t*    bm_create_model(bm_context_t* ctx, const bm_arch_t* arch);
void           bm_destroy_model(bm_model_t* model);

/* Reference include/baremetal.h:127: weights from a checkpoint directory
 * (config.json + model.safetensors, or shards listed by
 * model.safetensors.index.json; F32 or BF16 tensors, llama tensor names).
 * The model must have the shape config.json describes; errors are logged. */
void           bm_load_weights(bm_model_t* model, const char* path);

/* Uploads the weights and packs every projection to Q8 on the device
 * (the reference quantizes on the host at session creation,
 * reference src/baremetal/scheduler.c:364-384). */
void           bm_compile(bm_model_t* model);

bm_session_t*  bm_create_session(bm_context_t* ctx, bm_model_t* model);
/* Logits of the token at the session's position (V floats, valid until the
 * next call on the session); the position advances.  NULL on error. */
float*         bm_step(bm_session_t* sess, int token);
float*         bm_forward(bm_session_t* sess, const int* tokens, int n_tokens);
void           bm_reset_session(bm_session_t* sess);
void           bm_destroy_session(bm_session_t* sess);

/* GPU time of the steps run between begin and end, split as the reference
 * declares it: attention block (RMSNorm + q/k/v, RoPE + KV append +
 * attention, o + residual), MLP block (RMSNorm + gate/up + SwiGLU, down +
 * residual) and other (embedding, final norm + LM head + argmax).  The
 * reference declares the split but fills only other_ms (reference
 * src/baremetal/scheduler.c:994).  While profiling, steps are launched one
 * kernel at a time with a HIP event after each kernel (no graph replay). */
void           bm_profile_begin(bm_session_t* sess);
void           bm_profile_end(bm_session_t* sess, double* attention_ms, double* mlp_ms, double* other_ms);

typedef int (*bm_token_cb_t)(int token_id, void* user_data);

/* Reference tools/run.c:121-185: step every prompt token, then feed back
 * the sampled token; temperature <= 0 picks the first maximal logit.
 * Returns 0, or -1 on bad arguments. */
int            bm_run_tokens(bm_context_t* ctx, bm_model_t* model, const int* prompt_ids, int n_prompt, int steps,
                             float temperature, int top_k, float top_p, uint64_t seed, bm_token_cb_t callback,
                             void* user_data);

/* Reference src/baremetal/sampler.c: temperature -> softmax -> top-k ->
 * top-p -> inverse-CDF draw with an LCG; temperature <= 0 is argmax. */
bm_sampler_t*  bm_create_sampler(int vocab_size, float temp, float topp, uint64_t seed);
int            bm_sample(bm_sampler_t* sampler, const float* logits);
void           bm_destroy_sampler(bm_sampler_t* sampler);

int            bm_get_num_parameters(const bm_model_t* model);
const char*    bm_get_arch_name(const bm_model_t* model);

/* ---- MI355X additions (no reference counterpart) ---- */

/* Quantization of the projections: 8 (Q8_0, default) or 4 (Q4_0); the
 * reference's CLI sets model->quant_bits (reference tools/cli.c:886).
 * Returns 0, or -1 for another value. */
int            bm_model_set_quant_bits(bm_model_t* model, int bits);
/* 1: the LM head runs on Q8 rows quantized from the head (the tied embedding or lm_head);
 * 0 (default): rows in the model's precision, as the reference. */
int            bm_model_set_q8_head(bm_model_t* model, int on);
/* The reference's CLI writes model->precision after loading (reference
 * tools/cli.c:519-524); bm_model_t is opaque here, so this sets it.
 * BM_PRECISION_FP32 or BM_PRECISION_BF16; returns 0, or -1. */
int            bm_model_set_precision(bm_model_t* model, bm_precision_t precision);

/* Host fp32 weights in the reference's layout (reference
 * src/baremetal/model.c:125-172: one array per matrix type, layers back to
 * back, rows of the output dimension).  Names and element counts:
 *   "token_embedding" V*D   "ln1" L*D   "ln2" L*D   "lnf" D
 *   "wq" L*NH*HD*D  "wk" L*KV*D  "wv" L*KV*D  "wo" L*D*NH*HD
 *   "w_gate" L*H*D  "w_up" L*H*D  "w_down" L*D*H
 *   "lm_head" V*D (untied models only, weight_tie 0)
 * Returns 0, or -1 for an unknown name or a wrong count. */
int            bm_model_set_tensor(bm_model_t* model, const char* name, const float* data, size_t n);

/* bf16 weights (a checkpoint's raw tensor): projections stay bf16 until
 * bm_compile packs them to Q8 on the device from bf16 (the reference's
 * bmt_quantize_q8_bf16); other tensors are widened exactly.  Same names. */
int            bm_model_set_tensor_bf16(bm_model_t* model, const char* name, const uint16_t* data, size_t n);

/* A model from a Hugging Face checkpoint directory: config.json gives the
 * arch (reference src/baremetal/config.c:128-297; no lm_head tensor means a
 * tied head), then bm_load_weights.  NULL (logged) on error. */
bm_model_t*    bm_load_model(bm_context_t* ctx, const char* path);

/* The arch bm_load_model would build from a checkpoint directory, without
 * reading the tensors' data (host only).  Returns 0, or -1. */
int            bm_arch_from_checkpoint(const char* path, bm_arch_t* arch);

/* The model's arch as created. */
int            bm_model_arch(const bm_model_t* model, bm_arch_t* arch);

/* Random-init weights (no checkpoint): every projection of every layer and
 * the tied embedding drawn from N(0, 0.02) with the seed
 * bm_synth_tensor_seed(seed, 5, layer, id) (include/bm_synth.h), id =
 * 0 token_embedding (layer 0xFFFF), 1 wq, 2 wk, 3 wv, 4 wo, 5 w_gate,
 * 6 w_up, 7 w_down, 8 lm_head of an untied model (layer 0xFFFF);
 * RMSNorm gains 1.0. */
int            bm_model_init_synthetic(bm_model_t* model, uint64_t seed);

/* A session that steps `batch` independent sequences in lockstep (all at
 * the same position) with per-sequence KV caches; max_seq_len 0 takes the
 * model's.  bm_create_session is batch 1. */
bm_session_t*  bm_create_session_batched(bm_context_t* ctx, bm_model_t* model, int batch, int max_seq_len);

/* One step of every sequence: tokens[b] in, logits [batch][V] out. */
float*         bm_step_batch(bm_session_t* sess, const int* tokens);

/* Greedy generation driven on the device: from position 0, the prompt
 * prompt[b * n_prompt + i] is fed, then each sequence's argmax (first
 * maximal index) is fed back, for `steps` positions in total; no host
 * round trip between steps (the step is a replayed hipGraph).  Writes
 * steps - n_prompt + 1 tokens per sequence to out_tokens[i * batch + b]
 * (the same tokens bm_run_tokens emits) and returns that count, or -1. */
int            bm_generate_greedy(bm_session_t* sess, const int* prompt, int n_prompt, int steps, int* out_tokens);

/* 0: launch the step's kernels one by one instead of replaying the
 * captured graph (same kernels, same results).  Default 1. */
int            bm_session_set_graph(bm_session_t* sess, int on);

/* 1 (default where available): a session with Q8 projections on MI355X
 * and a batch of up to 16, or an even batch up to 32, runs every layer of a
 * decode step as one persistent kernel: instances of 32 workgroups, each on
 * one XCD running one or two sequences through five phases per layer that
 * hand values over without grid barriers; 0: one kernel per fused phase.
 * Both compute the same formulas in fp32 (summation orders differ).
 * Returns 0, or -1 when the persistent form is not available for the
 * session (then only 0 is accepted). */
int            bm_session_set_persistent(bm_session_t* sess, int on);

/* GPU time (HIP events around each submission) and submissions of the
 * session's host-driven steps and one-pass prefills, the counterpart of the
 * reference backend's busy time and command-buffer count
 * (reference src/backend/backend.h:32-35); reset != 0 zeroes both after
 * reading.  Returns 0, or -1. */
int            bm_session_gpu_stats(bm_session_t* sess, double* busy_ms, unsigned long long* launches, int reset);

/* Per-kernel-kind GPU ms accumulated since bm_profile_begin, in step order:
 * [0] embedding, [1] RMSNorm + q/k/v, [2] RoPE + KV append + attention,
 * [3] o + residual, [4] RMSNorm + gate/up + SwiGLU, [5] down + residual,
 * [6] final norm + LM head + argmax, [7] every layer as one persistent
 * kernel (batch-1 sessions that use it; [1]..[5] are then 0).  Returns the
 * number of profiled steps. */
#define BM_PROF_PHASES 8
long           bm_profile_phases(bm_session_t* sess, double* ms);

/* No counterpart in the reference.  For callers that cannot allocate device
 * memory (serving loops and harnesses that forbid hipMalloc once running):
 * bm_forward's one-pass prefill of a prompt at position 0 of a batch-1
 * session, with the same kernels and results, whose workspace (residual
 * stream, q/k/v rows, bf16 GEMM operands, norm sums, RoPE table, tokens)
 * lives in a static array of BM_NOALLOC_SCRATCH_BYTES per GPU instead of session
 * buffers allocated on the first prefill.  It calls no hipMalloc/hipFree and
 * allocates no host memory.  Like bm_forward it synchronizes the session's
 * stream and copies the logits back to the host, so it cannot be recorded
 * under HIP stream capture.  The caller passes the session (already
 * created), the tokens, and reads the logits returned (the session's
 * [V] floats, as bm_forward).  Rejects, with NULL and an error logged, a
 * prompt whose workspace exceeds the array (about 14 KB per token at
 * SmolLM2-135M shapes: at most about 4,700 tokens there), a session past
 * position 0 or with batch > 1, and n_tokens < 2.  Every call on one GPU
 * shares that GPU's array, so the library serializes bm_forward_noalloc
 * calls with one process-wide lock held until
 * the call returns: concurrent calls (other threads, other sessions or
 * GPUs) wait for each other rather than race. */
#define BM_NOALLOC_SCRATCH_BYTES (64u << 20)
float*         bm_forward_noalloc(bm_session_t* sess, const int* tokens, int n_tokens);

/* No counterpart in the reference; for tests only.  Forces the persistent
 * step kernel's failure paths from the host, every kernel still exiting
 * normally: mode 1, every wait for a value another workgroup exchanges
 * gives up after one tick (as a timeout would); mode 2, one working
 * workgroup acts as if placed on another XCD than its peers; mode 0, neither.  A step the
 * kernel flags void is rerun on the per-phase kernels, which the session
 * then keeps.  Returns the session's persistent state (0 not available,
 * 1 in use, 2 per-phase kernels in use), -1 on bad arguments, and in
 * *fallbacks (if not NULL) the number of steps rerun so far. */
int            bm_session_persist_test_fault(bm_session_t* sess, int mode, unsigned long long* fallbacks);

#ifdef __cplusplus
}
#endif

#endif /* BAREMETAL_H */
