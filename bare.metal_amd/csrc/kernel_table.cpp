/* SPDX-License-Identifier: MPL-2.0
 *
 * kernel_table.cpp — the named gfx950 kernels the HIP backend resolves in
 * backend_kernel_create.  Names and buffer orders follow the reference's
 * Metal kernels where one exists (cited per entry); the rest are MI355X
 * additions whose buffer orders are documented in include/bm_q8.h.
 *
 * Columns: name, buffers bound, by-value buffer mask, written buffer mask.
 */
#include "bmk.h"

extern "C" {
int bmk_launch_quantize_q8(const bmk_launch_t* a);
int bmk_launch_quantize_q8_bf16(const bmk_launch_t* a);
int bmk_launch_quantize_q4(const bmk_launch_t* a);
int bmk_launch_quantize_q4_bf16(const bmk_launch_t* a);
int bmk_launch_q4_matvec(const bmk_launch_t* a);
int bmk_launch_q4_matvec_multi(const bmk_launch_t* a);
int bmk_launch_q4_gemm_multi(const bmk_launch_t* a);
int bmk_launch_q8_matvec(const bmk_launch_t* a);
int bmk_launch_q8_matmul(const bmk_launch_t* a);
int bmk_launch_q8_matvec_multi(const bmk_launch_t* a);
int bmk_launch_copy_buffer(const bmk_launch_t* a);
int bmk_launch_stream_read(const bmk_launch_t* a);
int bmk_launch_mfma_ceiling(const bmk_launch_t* a);
int bmk_launch_q8_gemm_multi(const bmk_launch_t* a);
int bmk_launch_cast_bf16(const bmk_launch_t* a);
int bmk_launch_cast_bf16_frag(const bmk_launch_t* a);
int bmk_launch_rmsnorm(const bmk_launch_t* a);
int bmk_launch_rope(const bmk_launch_t* a);
int bmk_launch_kv_store(const bmk_launch_t* a);
int bmk_launch_attention(const bmk_launch_t* a);
int bmk_launch_attention_prefill(const bmk_launch_t* a);
int bmk_launch_rope_seq(const bmk_launch_t* a);
int bmk_launch_add(const bmk_launch_t* a);
int bmk_launch_swiglu(const bmk_launch_t* a);
int bmk_launch_rmsnorm_matmul(const bmk_launch_t* a);
int bmk_launch_rmsnorm_matmul_bf16(const bmk_launch_t* a);
int bmk_launch_rmsnorm_matmul_fp16(const bmk_launch_t* a);
int bmk_launch_argmax(const bmk_launch_t* a);
int bmk_launch_matmul_f32(const bmk_launch_t* a);
int bmk_launch_matmul_bf16(const bmk_launch_t* a);
int bmk_launch_matmul_fp16(const bmk_launch_t* a);
}

#define B(i) (1u << (i))

extern "C" const bmk_desc_t bmk_table[] = {
    /* new: the host loop of reference quant.c:54-71 as a device kernel;
     * {src f32, dst q8, params{n}} */
    {"quantize_q8", 3, B(2), B(1), bmk_launch_quantize_q8},
    /* new: reference quant.c:62-71 (bf16 source); {src bf16, dst q8, params{n}} */
    {"quantize_q8_bf16", 3, B(2), B(1), bmk_launch_quantize_q8_bf16},
    /* reference forward.metal:575-623; {inp, weight, bias, out, params{BT,C,OC,has_bias}} */
    {"matmul_forward_q8_vec", 5, B(4), B(3), bmk_launch_q8_matvec},
    /* reference forward.metal:625-649; same buffers */
    {"matmul_forward_q8", 5, B(4), B(3), bmk_launch_q8_matmul},
    /* Q4_0 (reference quant.c:31-52, forward.metal:654-858): new pack kernels
     * {src, dst q4, params{n}}; the reference's three matvec kernels, routed as
     * scheduler.c:755-764, buffers as the Q8 ones */
    {"quantize_q4", 3, B(2), B(1), bmk_launch_quantize_q4},
    {"quantize_q4_bf16", 3, B(2), B(1), bmk_launch_quantize_q4_bf16},
    {"matmul_forward_q4_vec4", 5, B(4), B(3), bmk_launch_q4_matvec},
    {"matmul_forward_q4_vec", 5, B(4), B(3), bmk_launch_q4_matvec},
    {"matmul_forward_q4", 5, B(4), B(3), bmk_launch_q4_matvec},
    /* new: every Q4 matvec of a decode token in one launch (plan: bm_q4_mv_plan) */
    {"matmul_forward_q4_vec_multi", 5, B(0) | B(1), B(4), bmk_launch_q4_matvec_multi, B(1)},
    /* new: many prefill GEMMs over Q4_0 weights in one launch (as matmul_forward_q8_multi) */
    {"matmul_forward_q4_multi", 5, B(0) | B(1), B(4), bmk_launch_q4_gemm_multi, B(1)},
    /* new: every Q8 matvec of a decode token in one launch; {params{nprob,n_tiles},
     * plan{MvDesc[nprob], u32 tile_map[n_tiles]}, weight arena, x arena, y arena} */
    {"matmul_forward_q8_vec_multi", 5, B(0) | B(1), B(4), bmk_launch_q8_matvec_multi, B(1)},
    /* new: many prefill GEMMs (bf16 MFMA) in one launch; {params{nprob,n_tiles},
     * plan{GmDesc[nprob], u32 tile_map[n_tiles]}, A arena, weight arena, C arena} */
    {"matmul_forward_q8_multi", 5, B(0) | B(1), B(4), bmk_launch_q8_gemm_multi, B(1)},
    /* new: fp32 -> bf16 activation cast (RNE); {src, dst, params int64{n}} */
    {"cast_f32_bf16", 3, B(2), B(1), bmk_launch_cast_bf16, 0},
    /* new: fp32 -> bf16 (RNE) into MFMA fragment order (matmul_forward_q8_multi layout 2);
     * {src f32 [M][lda], dst, params int{M, K, lda}} */
    {"cast_f32_bf16_frag", 3, B(2), B(1), bmk_launch_cast_bf16_frag, 0},
    /* new: device-to-device copy; {src, dst, params int64{nbytes}} */
    {"copy_buffer", 3, B(2), B(1), bmk_launch_copy_buffer, 0},
    /* new: read-only stream (HBM read ceiling); {src, sink u32[4*wg], params int64{nbytes, wg}} */
    {"stream_read", 3, B(2), B(1), bmk_launch_stream_read, 0},
    /* new: bf16 matrix-core rate (mode 0 register operands, 1 the GEMM's LDS-fed 2x2 wave tile);
     * {sink f32[256*wg], params int{wg, iters, mode}} */
    {"mfma_ceiling", 2, B(1), B(0), bmk_launch_mfma_ceiling, 0},
    /* decode-step kernels (buffer orders: reference scheduler.c:835-947) */
    /* reference forward.metal:1019-1060; {inp, weight, out, params{N,C}, eps} */
    {"rmsnorm_forward_v2", 5, B(3) | B(4), B(2), bmk_launch_rmsnorm, 0},
    /* reference forward.metal:1284-1313; {q, k, head_size, pos, rope[6], n_kv_heads}, grid = NH */
    {"rope_forward", 6, B(2) | B(3) | B(4) | B(5), B(0) | B(1), bmk_launch_rope, 0},
    /* reference forward.metal:1317-1329; {kv cache, k, v, params{layer,pos,MS,KV}} */
    {"kv_store", 4, B(3), B(0), bmk_launch_kv_store, 0},
    /* reference forward.metal:1362-1465; {q, kv cache, out, params{NH,HD,NKV,KV,S,kv_mul,layer,MS}, scale} */
    {"attention_forward", 5, B(3) | B(4), B(2), bmk_launch_attention, 0},
    /* reference forward.metal:2218-2257, prefill RoPE (scheduler.c:1097-1098);
     * {q [S][NH][HD], k [S][NKV][HD], params{head_size,n_kv_heads,S,NH}, rope[6]} */
    {"rope_forward_seq", 4, B(2) | B(3), B(0) | B(1), bmk_launch_rope_seq, 0},
    /* reference forward.metal:1904-2114, prefill attention (scheduler.c:1081-1089);
     * {Q [S][NH][HD] roped, K [S][NKV][HD], V, out [S][NH][HD], params{NH,S,HD,NKV,kv_mul}, scale} */
    {"attention_forward_prefill", 6, B(4) | B(5), B(3), bmk_launch_attention_prefill, 0},
    {"attention_forward_prefill_warp", 6, B(4) | B(5), B(3), bmk_launch_attention_prefill, 0},
    {"attention_forward_prefill_tiled", 6, B(4) | B(5), B(3), bmk_launch_attention_prefill, 0},
    /* reference forward.metal:1802-1848, the same causal attention over [S][NH][HD]
     * (the prefill fallback, scheduler.c:1089-1090); the reference caps S at 256 */
    {"attention_forward_seq", 6, B(4) | B(5), B(3), bmk_launch_attention_prefill, 0},
    /* reference forward.metal:1332-1340; {a, b, out, n} */
    {"add_forward", 4, B(3), B(2), bmk_launch_add, 0},
    /* reference forward.metal:1179-1190; {gate, up, out, N} */
    {"swiglu_forward", 4, B(3), B(2), bmk_launch_swiglu, 0},
    /* reference forward.metal:1636-1689; {x, norm weight, wcls f32, logits, params{C,V}, eps} */
    {"rmsnorm_matmul_forward", 6, B(4) | B(5), B(3), bmk_launch_rmsnorm_matmul, 0},
    /* reference forward.metal:1532-1581 (the LM head at default bf16 precision,
     * scheduler.c:776-778); {x, norm weight, wcls bf16, logits, params{C,V}, eps} */
    {"rmsnorm_matmul_forward_bf16_vec", 6, B(4) | B(5), B(3), bmk_launch_rmsnorm_matmul_bf16, 0},
    /* reference forward.metal:1691-1735, the same head with one thread per row
     * (scheduler.c:782-783 takes it at bf16 precision); same buffers and launch */
    {"rmsnorm_matmul_forward_bf16", 6, B(4) | B(5), B(3), bmk_launch_rmsnorm_matmul_bf16, 0},
    /* reference forward.metal:1585-1634 and 1748-1801: the same heads over fp16
     * rows (scheduler.c:779-785 takes them at fp16 precision); same buffers */
    {"rmsnorm_matmul_forward_fp16_vec", 6, B(4) | B(5), B(3), bmk_launch_rmsnorm_matmul_fp16, 0},
    {"rmsnorm_matmul_forward_fp16", 6, B(4) | B(5), B(3), bmk_launch_rmsnorm_matmul_fp16, 0},
    /* the plain fp32 / bf16 / fp16-weight matmuls, which the reference's
     * scheduler takes for unquantized projections and its prefill for the LM
     * head of the last position (graph.c:373-380, scheduler.c:764-775,
     * 1117-1141, registry.c:60-67): reference forward.metal:23-37, 513-560,
     * 449-503 (fp32), 52-89, 91-110, 116-319 (bf16), 327-442 (fp16);
     * {inp, weight, bias, out, params{BT,C,OC,has_bias}} */
    {"matmul_forward_naive", 5, B(4), B(3), bmk_launch_matmul_f32, 0},
    {"matmul_forward_tiled", 5, B(4), B(3), bmk_launch_matmul_f32, 0},
    {"matmul_forward_fp32_tiled", 5, B(4), B(3), bmk_launch_matmul_f32, 0},
    {"matmul_forward_bf16_vec", 5, B(4), B(3), bmk_launch_matmul_bf16, 0},
    {"matmul_forward_bf16", 5, B(4), B(3), bmk_launch_matmul_bf16, 0},
    {"matmul_forward_bf16_tiled", 5, B(4), B(3), bmk_launch_matmul_bf16, 0},
    {"matmul_forward_bf16_tiled64", 5, B(4), B(3), bmk_launch_matmul_bf16, 0},
    {"matmul_forward_bf16_simd", 5, B(4), B(3), bmk_launch_matmul_bf16, 0},
    {"matmul_forward_fp16_vec", 5, B(4), B(3), bmk_launch_matmul_fp16, 0},
    {"matmul_forward_fp16", 5, B(4), B(3), bmk_launch_matmul_fp16, 0},
    {"matmul_forward_fp16_tiled", 5, B(4), B(3), bmk_launch_matmul_fp16, 0},
    /* new: greedy pick on the device (reference tools/run.c:56-60); {values, out int, params{n}} */
    {"argmax_f32", 3, B(2), B(1), bmk_launch_argmax, 0},
    {nullptr, 0, 0, 0, nullptr, 0},
};
