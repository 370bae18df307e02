/* SPDX-License-Identifier: MPL-2.0
 *
 * synth.c — deterministic synthetic inputs for the benchmark configurations
 * and random-init models (there are no checkpoints in this setting).
 *
 * Element i of a tensor with seed s is a function of (s, i) only, so the
 * result does not depend on the thread count:
 *   chunk c = i / 4096 uses xoshiro256** seeded by four SplitMix64 draws
 *   from s ^ (c * 0x9E3779B97F4A7C15); consecutive pairs of its outputs
 *   become two N(0,1) values by the Box–Muller transform in double
 *   (u in (0,1] from the top 53 bits), scaled by sigma and rounded to fp32.
 * Everything runs on the host (never on the device), so the CPU oracle and
 * the GPU path consume bit-identical inputs.
 */
#include "bm_synth.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

#define SYN_CHUNK 4096

static uint64_t splitmix64(uint64_t* s) {
    uint64_t z = (*s += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

typedef struct { uint64_t s[4]; } xo256_t;

static inline uint64_t rotl64(uint64_t x, int k) { return (x << k) | (x >> (64 - k)); }

static uint64_t xo_next(xo256_t* x) {
    uint64_t* s = x->s;
    const uint64_t r = rotl64(s[1] * 5, 7) * 9;
    const uint64_t t = s[1] << 17;
    s[2] ^= s[0];
    s[3] ^= s[1];
    s[1] ^= s[2];
    s[0] ^= s[3];
    s[2] ^= t;
    s[3] = rotl64(s[3], 45);
    return r;
}

static void xo_seed(xo256_t* x, uint64_t seed, uint64_t chunk) {
    uint64_t sm = seed ^ (chunk * 0x9E3779B97F4A7C15ull);
    for (int i = 0; i < 4; i++) x->s[i] = splitmix64(&sm);
}

static inline double unit_open0(uint64_t r) {
    /* (0, 1]: never 0, so log() is finite */
    return ((double)(r >> 11) + 1.0) * (1.0 / 9007199254740992.0);
}

uint64_t bm_synth_tensor_seed(uint64_t base, int model_id, int layer, int matrix_id) {
    uint64_t s = base ^ ((uint64_t)(uint32_t)model_id << 40) ^ ((uint64_t)(uint32_t)layer << 16) ^ (uint64_t)(uint32_t)matrix_id;
    return splitmix64(&s);
}

static void normal_chunks(uint64_t seed, float sigma, float* out, size_t n, size_t c0, size_t c1) {
    const double two_pi = 6.283185307179586476925286766559;
    for (size_t c = c0; c < c1; c++) {
        xo256_t x;
        xo_seed(&x, seed, (uint64_t)c);
        size_t i0 = c * SYN_CHUNK, i1 = i0 + SYN_CHUNK;
        if (i1 > n) i1 = n;
        for (size_t i = i0; i < i1; i += 2) {
            double u1 = unit_open0(xo_next(&x));
            double u2 = unit_open0(xo_next(&x));
            double r = sqrt(-2.0 * log(u1));
            double th = two_pi * u2;
            out[i] = (float)((double)sigma * r * cos(th));
            if (i + 1 < i1) out[i + 1] = (float)((double)sigma * r * sin(th));
        }
    }
}

typedef struct {
    uint64_t seed;
    float sigma;
    float* out;
    size_t n, c0, c1;
} syn_job_t;

static void* syn_worker(void* p) {
    syn_job_t* j = (syn_job_t*)p;
    normal_chunks(j->seed, j->sigma, j->out, j->n, j->c0, j->c1);
    return NULL;
}

static int syn_threads(void) {
    const char* e = getenv("BM_SYNTH_THREADS");
    int t = (e && e[0]) ? atoi(e) : 16;
    if (t < 1) t = 1;
    if (t > 64) t = 64;
    return t;
}

void bm_synth_normal_f32(uint64_t seed, float sigma, float* out, size_t n) {
    if (!out || n == 0) return;
    size_t nchunks = (n + SYN_CHUNK - 1) / SYN_CHUNK;
    int nt = syn_threads();
    if (nchunks < 64 || nt == 1) {
        normal_chunks(seed, sigma, out, n, 0, nchunks);
        return;
    }
    if ((size_t)nt > nchunks) nt = (int)nchunks;
    pthread_t th[64];
    syn_job_t jobs[64];
    int started = 0;
    for (int k = 0; k < nt; k++) {
        jobs[k].seed = seed;
        jobs[k].sigma = sigma;
        jobs[k].out = out;
        jobs[k].n = n;
        jobs[k].c0 = nchunks * (size_t)k / (size_t)nt;
        jobs[k].c1 = nchunks * (size_t)(k + 1) / (size_t)nt;
        if (pthread_create(&th[k], NULL, syn_worker, &jobs[k]) == 0) {
            started = k + 1;
        } else {
            /* no thread: do this share (and every later one) here */
            for (int r = k; r < nt; r++) {
                size_t a0 = nchunks * (size_t)r / (size_t)nt, a1 = nchunks * (size_t)(r + 1) / (size_t)nt;
                normal_chunks(seed, sigma, out, n, a0, a1);
            }
            break;
        }
    }
    for (int k = 0; k < started; k++) pthread_join(th[k], NULL);
}

void bm_synth_uniform_int(uint64_t seed, int lo, int hi, int* out, size_t n) {
    if (!out || n == 0 || hi <= lo) return;
    const uint64_t range = (uint64_t)((int64_t)hi - (int64_t)lo);
    xo256_t x;
    xo_seed(&x, seed, 0);
    for (size_t i = 0; i < n; i++) {
        /* 64x64->128 multiply-shift: uniform up to 2^-64 bias */
        unsigned __int128 m = (unsigned __int128)xo_next(&x) * range;
        out[i] = lo + (int)(uint64_t)(m >> 64);
    }
}

void bm_synth_fill_f32(float value, float* out, size_t n) {
    for (size_t i = 0; i < n; i++) out[i] = value;
}
