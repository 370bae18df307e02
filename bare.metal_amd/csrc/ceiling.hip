/* SPDX-License-Identifier: MPL-2.0
 *
 * ceiling.hip — the bf16 matrix-core rate this part reaches, as a named
 * kernel ("mfma_ceiling"), reported beside the prefill GEMM's MFMA fraction
 * as stream_read is beside the matvec's bandwidth.
 *
 *   mode 0: each wave runs 8 independent v_mfma_f32_32x32x16_bf16
 *           accumulator chains on register operands (no memory traffic):
 *           the matrix pipe's own rate;
 *   mode 1: each wave reads its operands from LDS per 16-deep K slice as the
 *           prefill GEMM's inner loop does (a 64x64 wave tile = 2x2 MFMA tiles,
 *           two A and two B fragments of 16 bytes per lane per slice, rows
 *           padded to 72 bf16), with the rows moving every iteration so
 *           that no read can be hoisted: the rate of that tiling with no
 *           global traffic, no dequantisation and no barrier.
 *
 * Each lane writes one sum of its accumulators to sink so that no MFMA is
 * dead.  FLOPs per launch: workgroups x 4 waves x iters x 8 x 32768.
 */
#include "bmk.h"

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int CE_LDK = 72; /* LDS row in bf16 elements, as the GEMM's slabs */

__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void k_mfma_regs(float* __restrict__ sink,
                                                                                              int iters) {
    bf16x8 a, b;
    for (int i = 0; i < 8; i++) {
        a[i] = (__bf16)(1e-3f * (float)(threadIdx.x + i));
        b[i] = (__bf16)(1e-3f * (float)(8 - i));
    }
    f32x16 acc[8];
    for (int c = 0; c < 8; c++)
        for (int r = 0; r < 16; r++) acc[c][r] = 0.f;
    for (int it = 0; it < iters; it++) {
#pragma unroll
        for (int c = 0; c < 8; c++) acc[c] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, acc[c], 0, 0, 0);
    }
    float s = 0.f;
    for (int c = 0; c < 8; c++)
        for (int r = 0; r < 16; r++) s += acc[c][r];
    sink[(size_t)blockIdx.x * 256 + threadIdx.x] = s;
}

/* 2x2 tiles per wave, two K slices of 16 per iteration (8 MFMAs) */
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void k_mfma_lds(float* __restrict__ sink,
                                                                                             int iters) {
    __shared__ __attribute__((aligned(16))) unsigned short lds[2 * 128 * CE_LDK];
    for (int i = threadIdx.x; i < 2 * 128 * CE_LDK; i += 256) lds[i] = (unsigned short)(0x3a80 + (i & 15));
    __syncthreads();
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wm = (wave >> 1) * 64, wn = (wave & 1) * 64, kq = (lane >> 5) * 8;
    const unsigned short* As = lds;
    const unsigned short* Bs = lds + 128 * CE_LDK;
    f32x16 acc[2][2];
    for (int i = 0; i < 2; i++)
        for (int j = 0; j < 2; j++)
            for (int r = 0; r < 16; r++) acc[i][j][r] = 0.f;
    for (int it = 0; it < iters; it++) {
        const int rot = (it * 8) & 127;
        const int ks0 = (it & 1) * 32;
#pragma unroll
        for (int ks = ks0; ks < ks0 + 32; ks += 16) {
            bf16x8 fa[2], fb[2];
#pragma unroll
            for (int i = 0; i < 2; i++) fa[i] = *(const bf16x8*)&As[((wm + 32 * i + (lane & 31) + rot) & 127) * CE_LDK + ks + kq];
#pragma unroll
            for (int j = 0; j < 2; j++) fb[j] = *(const bf16x8*)&Bs[((wn + 32 * j + (lane & 31) + rot) & 127) * CE_LDK + ks + kq];
#pragma unroll
            for (int i = 0; i < 2; i++)
#pragma unroll
                for (int j = 0; j < 2; j++) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[i], fb[j], acc[i][j], 0, 0, 0);
        }
    }
    float s = 0.f;
    for (int i = 0; i < 2; i++)
        for (int j = 0; j < 2; j++)
            for (int r = 0; r < 16; r++) s += acc[i][j][r];
    sink[(size_t)blockIdx.x * 256 + threadIdx.x] = s;
}

} // namespace

/* mfma_ceiling {0 sink f32 [256 * workgroups], 1 params int{workgroups, iters, mode}} */
extern "C" int bmk_launch_mfma_ceiling(const bmk_launch_t* a) {
    BMK_NEED_BYTES(a, 1, 12, "params");
    const int wg = bmk_pi(a, 1, 0), iters = bmk_pi(a, 1, 1), mode = bmk_pi(a, 1, 2);
    BMK_REQUIRE(wg > 0 && wg <= 65536 && iters > 0 && (mode == 0 || mode == 1),
                "mfma_ceiling: bad params workgroups=%d iters=%d mode=%d", wg, iters, mode);
    BMK_NEED_BYTES(a, 0, (size_t)wg * 256 * 4, "sink");
    float* sink = (float*)a->dev[0];
    if (mode == 0) hipLaunchKernelGGL(k_mfma_regs, dim3((unsigned)wg), dim3(256), 0, a->stream, sink, iters);
    else hipLaunchKernelGGL(k_mfma_lds, dim3((unsigned)wg), dim3(256), 0, a->stream, sink, iters);
    BMK_LAUNCH_CHECK();
    return 0;
}
