/* SPDX-License-Identifier: MPL-2.0
 *
 * oracle.h — CPU restatement of the reference's Q8 path (test
 * infrastructure only; see oracle.c).
 */
#ifndef BM_ORACLE_H
#define BM_ORACLE_H

#include <stddef.h>
#include <stdint.h>

size_t   orc_quantize_q8(const float* src, uint8_t* dst, size_t n);
size_t   orc_quantize_q8_bf16(const uint16_t* src, uint8_t* dst, size_t n);
uint16_t orc_bf16_rne(float f);
void     orc_bf16_round_array(const float* src, float* dst, size_t n);
void     orc_q8_matvec_f64(const uint8_t* w, const float* x, double* y, int BT, int C, int OC);
void     orc_q8_gemm_bf16_f64(const uint8_t* w, const float* a, double* c, int M, int K, int N);
size_t   orc_quantize_q4(const float* src, uint8_t* dst, size_t n);
size_t   orc_quantize_q4_bf16(const uint16_t* src, uint8_t* dst, size_t n);
void     orc_q4_matvec_f64(const uint8_t* w, const float* x, double* y, int BT, int C, int OC);
void     orc_q4_gemm_bf16_f64(const uint8_t* w, const float* a, double* c, int M, int K, int N);

/* CPU baseline (cpu_baseline.c): fp32 Q8 matvec in the reference's
 * arithmetic, SIMD + OpenMP over rows. */
void     orc_cpu_q8_matvec_f32(const uint8_t* w, const float* x, float* y, int C, int OC, int nthreads);
void     orc_cpu_q8_matvec_multi(const uint8_t* w, const float* x, float* y, int nprob, const uint64_t* w_off,
                                 const uint64_t* x_off, const uint64_t* y_off, const int* OC, const int* C,
                                 int nthreads);
int      orc_cpu_max_threads(void);
const char* orc_cpu_isa(void);
/* fp32 SIMD decoder (config-5 CPU baseline, cpu_baseline.c); m is an
 * orc_model_t (decode_oracle.h) with Q8 projections and an fp32 head. */
void*    orc_cpu_decoder_create(const void* m, int nthreads);
void     orc_cpu_decoder_destroy(void* d);
int      orc_cpu_decoder_step(void* d, int token, int pos, float* logits_out);

#endif
