/* SPDX-License-Identifier: MPL-2.0
 *
 * bm_synth.h — deterministic host-side synthetic data (no reference
 * counterpart: the reference loads real checkpoints).  Used to build the
 * benchmark configurations' N(0,0.02) weights, N(0,1) activations and
 * uniform prompt ids, identically for the GPU path and the CPU oracle.
 */
#ifndef BM_SYNTH_H
#define BM_SYNTH_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Per-tensor seed from a base seed and the tensor's identity. */
uint64_t bm_synth_tensor_seed(uint64_t base, int model_id, int layer, int matrix_id);

/* out[i] = fp32(sigma * N(0,1)) for i < n; a pure function of (seed, i). */
void bm_synth_normal_f32(uint64_t seed, float sigma, float* out, size_t n);

/* out[i] uniform in [lo, hi). */
void bm_synth_uniform_int(uint64_t seed, int lo, int hi, int* out, size_t n);

void bm_synth_fill_f32(float value, float* out, size_t n);

#ifdef __cplusplus
}
#endif

#endif
