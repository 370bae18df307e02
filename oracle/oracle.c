/* SPDX-License-Identifier: MPL-2.0
 *
 * oracle.c — CPU restatement of the reference's Q8 arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py load this library, and only as the checker
 * (or as the timed CPU baseline); the product library never links or calls
 * it.
 *
 * Every function cites the reference code it restates.  How each is pinned:
 *   orc_quantize_q8 / _bf16   bit-identical to the reference's own quant.c
 *                             compiled from /root/reference into oracle/_ref
 *                             (tests/test_oracle.py), committed golden bytes
 *                             made by that build (tests/golden/), and
 *                             closed-form special cases;
 *   orc_q8_matvec_f64         one-hot and integer-exact inputs against
 *                             closed forms, linearity, and a float128-free
 *                             brute-force re-sum in a different order;
 *   orc_q8_gemm_*             row-by-row agreement with orc_q8_matvec_f64
 *                             (exact variant) and a hand-worked bf16 case;
 *   orc_quantize_q4 / _bf16   as the Q8 pack: bit-identical to the
 *                             reference's quant.c in oracle/_ref, committed
 *                             golden bytes, closed-form special cases;
 *   orc_q4_matvec_f64         one-hot and integer-exact inputs against
 *                             closed forms, and agreement with the Q8 matvec
 *                             on weights whose Q8 and Q4 codes coincide;
 *   orc_bf16_rne              the reference's bm_f32_to_bf16 bit trick,
 *                             checked against known roundings.
 * Parity of the Metal kernels' fp32 summation order is not pinnable (the
 * Metal compiler's fast-math order is undefined), so sums are compared with
 * tolerances; packing is compared bit for bit.
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ---- Q8 pack: reference src/baremetal/quant.c:10-29 (block), :54-60 (fp32 loop),
 *      :62-71 (bf16 source), include/baremetal/types.h:15-20 (bf16 widening). */

static int orc_lround_int_clamp(float y) {
    /* (int)lroundf(y) clamped to [-128,127], as x86-64 glibc evaluates it:
     * lroundf of NaN / Inf returns LONG_MIN, whose conversion to int is 0. */
    if (isnan(y) || isinf(y)) return 0;
    double t = trunc((double)y);
    if (fabs((double)y - t) >= 0.5) t += (y < 0.0f) ? -1.0 : 1.0;
    if (t > 127.0) t = 127.0;
    if (t < -128.0) t = -128.0;
    return (int)t;
}

static void orc_quant_block(const float* p, uint8_t* dst) {
    float amax = 0.0f;
    for (int i = 0; i < 32; i++) {
        float a = fabsf(p[i]);
        if (a > amax) amax = a;
    }
    volatile float scale = amax / 127.0f; /* volatile: keep the fp32 rounding */
    float s = scale;
    memcpy(dst, &s, 4);
    if (s == 0.0f) {
        memset(dst + 4, 0, 32);
        return;
    }
    volatile float inv = 1.0f / s;
    float iv = inv;
    for (int i = 0; i < 32; i++) {
        volatile float y = p[i] * iv;
        dst[4 + i] = (uint8_t)(int8_t)orc_lround_int_clamp(y);
    }
}

size_t orc_quantize_q8(const float* src, uint8_t* dst, size_t n) {
    if (n == 0 || n % 32) return 0;
    for (size_t b = 0; b < n / 32; b++) orc_quant_block(src + 32 * b, dst + 36 * b);
    return n / 32;
}

size_t orc_quantize_q8_bf16(const uint16_t* src, uint8_t* dst, size_t n) {
    if (n == 0 || n % 32) return 0;
    float tmp[32];
    for (size_t b = 0; b < n / 32; b++) {
        for (int i = 0; i < 32; i++) {
            uint32_t u = (uint32_t)src[32 * b + i] << 16;
            memcpy(&tmp[i], &u, 4);
        }
        orc_quant_block(tmp, dst + 36 * b);
    }
    return n / 32;
}

/* ---- Q4 pack: reference src/baremetal/quant.c:31-52 (block; 20-byte
 *      {f32 scale; u8 qs[16]}, quant.h:34-42), :73-90 (fp32 / bf16 loops).
 *      Element 2j sits in the low nibble of qs[j], element 2j+1 in the high
 *      nibble, each a two's-complement 4-bit code in [-8, 7]. */

static int orc_lround_int_clamp4(float y) {
    if (isnan(y) || isinf(y)) return 0; /* (int)LONG_MIN, as above */
    double t = trunc((double)y);
    if (fabs((double)y - t) >= 0.5) t += (y < 0.0f) ? -1.0 : 1.0;
    if (t > 7.0) t = 7.0;
    if (t < -8.0) t = -8.0;
    return (int)t;
}

static void orc_quant4_block(const float* p, uint8_t* dst) {
    float amax = 0.0f;
    for (int i = 0; i < 32; i++) {
        float a = fabsf(p[i]);
        if (a > amax) amax = a;
    }
    volatile float scale = amax / 7.0f;
    float s = scale;
    memcpy(dst, &s, 4);
    if (s == 0.0f) {
        memset(dst + 4, 0, 16);
        return;
    }
    volatile float inv = 1.0f / s;
    float iv = inv;
    for (int j = 0; j < 16; j++) {
        volatile float y0 = p[2 * j] * iv;
        volatile float y1 = p[2 * j + 1] * iv;
        const int lo = orc_lround_int_clamp4(y0), hi = orc_lround_int_clamp4(y1);
        dst[4 + j] = (uint8_t)((lo & 0x0F) | ((hi & 0x0F) << 4));
    }
}

size_t orc_quantize_q4(const float* src, uint8_t* dst, size_t n) {
    if (n == 0 || n % 32) return 0;
    for (size_t b = 0; b < n / 32; b++) orc_quant4_block(src + 32 * b, dst + 20 * b);
    return n / 32;
}

size_t orc_quantize_q4_bf16(const uint16_t* src, uint8_t* dst, size_t n) {
    if (n == 0 || n % 32) return 0;
    float tmp[32];
    for (size_t b = 0; b < n / 32; b++) {
        for (int i = 0; i < 32; i++) {
            uint32_t u = (uint32_t)src[32 * b + i] << 16;
            memcpy(&tmp[i], &u, 4);
        }
        orc_quant4_block(tmp, dst + 20 * b);
    }
    return n / 32;
}

/* The signed 4-bit code of element j (0..31) of a Q4 block's qs[16]. */
static inline int q4_code(const uint8_t* qs, int j) {
    const int nib = (qs[j >> 1] >> (4 * (j & 1))) & 0x0F;
    return nib >= 8 ? nib - 16 : nib;
}

/* ---- Q4 matvec: reference forward.metal:654-858 (matmul_forward_q4_vec4,
 *      _vec, and the BT>1 matmul_forward_q4): y[bt][oc] = sum_b scale[oc][b] *
 *      sum_j x[bt][32b+j] * code[oc][b][j], exactly in double. */
void orc_q4_matvec_f64(const uint8_t* w, const float* x, double* y, int BT, int C, int OC) {
    const int nb = C / 32;
    for (int bt = 0; bt < BT; bt++) {
        const float* xr = x + (size_t)bt * C;
        for (int oc = 0; oc < OC; oc++) {
            const uint8_t* row = w + (size_t)oc * nb * 20;
            double acc = 0.0;
            for (int b = 0; b < nb; b++) {
                const uint8_t* blk = row + (size_t)b * 20;
                float sf;
                memcpy(&sf, blk, 4);
                double part = 0.0;
                for (int j = 0; j < 32; j++) part += (double)xr[32 * b + j] * (double)q4_code(blk + 4, j);
                acc += (double)sf * part;
            }
            y[(size_t)bt * OC + oc] = acc;
        }
    }
}

/* ---- bf16 cast: reference include/baremetal/types.h:22-29 (RNE bit trick). */
uint16_t orc_bf16_rne(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

static float bf16_to_f32(uint16_t h) {
    uint32_t u = (uint32_t)h << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

static inline float q8_scale(const uint8_t* blk) {
    float s;
    memcpy(&s, blk, 4);
    return s;
}

/* ---- Q8 matvec: reference forward.metal:575-623 (BT==1) and :625-649 (BT>1):
 *      y[bt][oc] = sum_b scale[oc][b] * sum_j x[bt][32b+j] * q[oc][b][j],
 *      evaluated exactly in double (every product of an fp32 x, an int8 q and
 *      an fp32 scale, and their sum, carried at 53 bits). */
void orc_q8_matvec_f64(const uint8_t* w, const float* x, double* y, int BT, int C, int OC) {
    const int nb = C / 32;
    for (int bt = 0; bt < BT; bt++) {
        const float* xr = x + (size_t)bt * C;
        for (int oc = 0; oc < OC; oc++) {
            const uint8_t* row = w + (size_t)oc * nb * 36;
            double acc = 0.0;
            for (int b = 0; b < nb; b++) {
                const uint8_t* blk = row + (size_t)b * 36;
                double s = (double)q8_scale(blk);
                double part = 0.0;
                for (int j = 0; j < 32; j++) part += (double)xr[32 * b + j] * (double)(int8_t)blk[4 + j];
                acc += s * part;
            }
            y[(size_t)bt * OC + oc] = acc;
        }
    }
}

/* ---- Prefill GEMM with bf16 operands (the MFMA contract):
 *      C[m][n] = sum_k bf16(A[m][k]) * bf16(q[n][k] * scale[n][k/32]) in double. */
/* C = A x Wd^T in double over bf16-rounded A; Wd: N rows of K dequantized
 * weights (already bf16 values).  Frees wd. */
static void contract_bf16_f64(float* wd, const float* a, double* c, int M, int K, int N) {
    float* ad = (float*)malloc((size_t)M * K * sizeof(float));
    if (!wd || !ad) {
        free(wd);
        free(ad);
        return;
    }
    for (size_t i = 0; i < (size_t)M * K; i++) ad[i] = bf16_to_f32(orc_bf16_rne(a[i]));
    for (int m = 0; m < M; m++)
        for (int n = 0; n < N; n++) {
            double acc = 0.0;
            const float* ar = ad + (size_t)m * K;
            const float* wr = wd + (size_t)n * K;
            for (int k = 0; k < K; k++) acc += (double)ar[k] * (double)wr[k];
            c[(size_t)m * N + n] = acc;
        }
    free(wd);
    free(ad);
}

void orc_q8_gemm_bf16_f64(const uint8_t* w, const float* a, double* c, int M, int K, int N) {
    const int nb = K / 32;
    float* wd = (float*)malloc((size_t)N * K * sizeof(float));
    for (int n = 0; wd && n < N; n++)
        for (int b = 0; b < nb; b++) {
            const uint8_t* blk = w + ((size_t)n * nb + b) * 36;
            float s = q8_scale(blk);
            for (int j = 0; j < 32; j++) {
                volatile float v = (float)(int8_t)blk[4 + j] * s;
                wd[(size_t)n * K + 32 * b + j] = bf16_to_f32(orc_bf16_rne(v));
            }
        }
    contract_bf16_f64(wd, a, c, M, K, N);
}

/* ---- Prefill GEMM over Q4_0 weights with bf16 operands: the same with
 *      bf16(code * scale) (reference forward.metal:829-858 at BT > 1). */
void orc_q4_gemm_bf16_f64(const uint8_t* w, const float* a, double* c, int M, int K, int N) {
    const int nb = K / 32;
    float* wd = (float*)malloc((size_t)N * K * sizeof(float));
    for (int n = 0; wd && n < N; n++)
        for (int b = 0; b < nb; b++) {
            const uint8_t* blk = w + ((size_t)n * nb + b) * 20;
            float s;
            memcpy(&s, blk, 4);
            for (int j = 0; j < 32; j++) {
                volatile float v = (float)q4_code(blk + 4, j) * s;
                wd[(size_t)n * K + 32 * b + j] = bf16_to_f32(orc_bf16_rne(v));
            }
        }
    contract_bf16_f64(wd, a, c, M, K, N);
}

/* fp32 activation rounded to bf16 and back (A10 semantics), elementwise. */
void orc_bf16_round_array(const float* src, float* dst, size_t n) {
    for (size_t i = 0; i < n; i++) dst[i] = bf16_to_f32(orc_bf16_rne(src[i]));
}
