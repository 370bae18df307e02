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
 * for the host: 8 independent fp32 partial sums per block so the compiler
 * vectorises it (AVX-512 / AVX2 / baseline x86-64 picked at load time by
 * target_clones), rows split over OpenMP threads.
 */
#include "oracle.h"

#include <omp.h>
#include <string.h>

__attribute__((target_clones("avx512f", "avx2", "default")))
static void rows_f32(const uint8_t* w, const float* x, float* y, int C, int r0, int r1) {
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
    if (__builtin_cpu_supports("avx512f")) return "avx512f";
    if (__builtin_cpu_supports("avx2")) return "avx2";
    return "x86-64";
}
