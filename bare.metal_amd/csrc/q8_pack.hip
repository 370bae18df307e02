/* SPDX-License-Identifier: MPL-2.0
 *
 * q8_pack.hip — fp32/bf16 -> Q8_0 (and Q4_0, below) block quantize/pack on
 * gfx950.
 *
 * Output format (reference src/baremetal/quant.h:17-32): an array of 36-byte
 * blocks {float scale; int8 q[32]}, block b covering source elements
 * 32b..32b+31.  Per block (reference src/baremetal/quant.c:10-29):
 *   amax  = max |p_i|   (strict '>' from 0, so NaN elements never win)
 *   scale = amax / 127.0f              (IEEE division, round to nearest)
 *   scale == 0  ->  every q_i = 0, stored scale = +0
 *   inv   = 1.0f / scale                (IEEE division)
 *   q_i   = clamp((int)lroundf(p_i * inv), -128, 127)
 * lroundf rounds half away from zero.  For finite blocks |p_i * inv| never
 * exceeds 127.0001, so the clamp never fires; p_i * inv is NaN or infinite
 * only when the block holds an Inf or when 1/scale overflows (scale below
 * 2^-128), and there x86-64's lroundf returns LONG_MIN, whose int conversion
 * is 0 — the value used here.
 *
 * The hardware division on this path is correctly rounded: the file is built
 * without fast-math, so '/' lowers to the v_div_scale/v_div_fmas/v_div_fixup
 * sequence, and fp32 denormals are kept.
 *
 * Mapping: 8 lanes per block, each lane owns 4 consecutive elements (one
 * 16-byte load), so a wave reads 1 KiB of contiguous source (8 blocks) per
 * load instruction.  The block max is a 3-step xor shuffle inside
 * the 8-lane group.  A Q8 workgroup packs 2 such 32-block groups, with both
 * source loads of a lane issued before the first reduction, and writes its
 * blocks from LDS as whole 16-byte stores.  HBM-bound: 4 (or 2) + 1.125
 * bytes per element.
 */
#include "bmk.h"

namespace {

__device__ __forceinline__ int q8_round_clamp(float y) {
    /* NaN or infinite -> 0 (see header). */
    if (!(fabsf(y) <= 3.402823466e38f)) return 0;
    float t = truncf(y);
    if (fabsf(y - t) >= 0.5f) t += copysignf(1.0f, y); /* y - t is exact */
    t = fminf(fmaxf(t, -128.0f), 127.0f);
    return (int)t;
}

template <bool SRC_BF16>
__device__ __forceinline__ void load4(const void* src, long e, float v[4]) {
    if (SRC_BF16) {
        const unsigned short* s = (const unsigned short*)src + e;
        uint2 raw;
        __builtin_memcpy(&raw, __builtin_assume_aligned(s, 8), 8);
        v[0] = __uint_as_float(raw.x << 16);
        v[1] = __uint_as_float(raw.x & 0xffff0000u);
        v[2] = __uint_as_float(raw.y << 16);
        v[3] = __uint_as_float(raw.y & 0xffff0000u);
    } else {
        const float* s = (const float*)src + e;
        float4 raw;
        __builtin_memcpy(&raw, __builtin_assume_aligned(s, 4), 16);
        v[0] = raw.x; v[1] = raw.y; v[2] = raw.z; v[3] = raw.w;
    }
}

/* One block's scale and this lane's 4 packed codes from the lane's 4
 * elements; the block max meets over the 8-lane group. */
__device__ __forceinline__ unsigned int q8_pack4(const float v[4], float& scale_out) {
    float m = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        float a = fabsf(v[i]);
        m = (a > m) ? a : m;
    }
#pragma unroll
    for (int off = 1; off < 8; off <<= 1) {
        float o = __shfl_xor(m, off, 8);
        m = (o > m) ? o : m;
    }
    const float scale = m / 127.0f;
    unsigned int packed = 0u;
    if (scale != 0.0f) {
        const float inv = 1.0f / scale;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            int q = q8_round_clamp(v[i] * inv);
            packed |= ((unsigned int)q & 0xffu) << (8 * i);
        }
    }
    scale_out = scale;
    return packed;
}

/* A workgroup packs PK_U groups of 32 consecutive blocks: step u covers
 * blocks (blockIdx.x * PK_U + u) * 32 + lane / 8.  Every step's source load
 * is issued before the first block is reduced; the loads are nontemporal
 * (the source is read once).  The workgroup's blocks (PK_U * 32 * 36 bytes,
 * one contiguous span) are assembled in LDS and written with 16-byte
 * nontemporal stores, so every destination line is written whole by one
 * instruction instead of in 4-byte pieces by two (codes, then scales).
 * Measured on the SmolLM2-360M weights against the direct 4-byte stores of
 * PK_U = 4 (launches interleaved on one part): 360M set 317 -> 284 us,
 * 49152x960 head 45.5 -> 44.2 us; PK_U = 2 beat 4 and 8 with this store
 * path.  ALIGNED: source 16-byte (bf16: 8-byte) and destination 16-byte
 * aligned; otherwise plain loads and 4-byte stores from LDS. */
constexpr int PK_U = 2;
constexpr int PK_WORDS = PK_U * 32 * 9; /* 36-byte blocks of a workgroup, in 4-byte words */

typedef float pk_f4 __attribute__((ext_vector_type(4)));
typedef unsigned int pk_u2 __attribute__((ext_vector_type(2)));
typedef unsigned int pk_u4 __attribute__((ext_vector_type(4)));

template <bool SRC_BF16, bool ALIGNED>
__device__ __forceinline__ void load4_stream(const void* src, long e, float v[4]) {
    if (!ALIGNED) {
        load4<SRC_BF16>(src, e, v);
    } else if (SRC_BF16) {
        const pk_u2 raw = __builtin_nontemporal_load((const pk_u2*)((const unsigned short*)src + e));
        v[0] = __uint_as_float(raw.x << 16);
        v[1] = __uint_as_float(raw.x & 0xffff0000u);
        v[2] = __uint_as_float(raw.y << 16);
        v[3] = __uint_as_float(raw.y & 0xffff0000u);
    } else {
        const pk_f4 raw = __builtin_nontemporal_load((const pk_f4*)((const float*)src + e));
        v[0] = raw.x; v[1] = raw.y; v[2] = raw.z; v[3] = raw.w;
    }
}

template <bool SRC_BF16, bool ALIGNED>
__global__ __launch_bounds__(256) void k_quantize_q8(const void* __restrict__ src, unsigned char* __restrict__ dst,
                                                     long nblocks) {
    __shared__ __attribute__((aligned(16))) unsigned int out[PK_WORDS];
    const int j = threadIdx.x & 7;
    const long wb = (long)blockIdx.x * (PK_U * 32);
    const long blk0 = wb + (threadIdx.x >> 3);
    float v[PK_U][4];
#pragma unroll
    for (int u = 0; u < PK_U; u++) {
        const long blk = blk0 + 32 * u;
        v[u][0] = v[u][1] = v[u][2] = v[u][3] = 0.0f;
        if (blk < nblocks) load4_stream<SRC_BF16, ALIGNED>(src, blk * 32 + 4 * j, v[u]);
    }
#pragma unroll
    for (int u = 0; u < PK_U; u++) {
        float scale;
        const unsigned int packed = q8_pack4(v[u], scale);
        const int lb = u * 32 + (threadIdx.x >> 3);
        out[lb * 9 + 1 + j] = packed;
        if (j == 0) out[lb * 9] = __float_as_uint(scale);
    }
    __syncthreads();
    const int nb = (int)min((long)(PK_U * 32), nblocks - wb);
    if (ALIGNED && nb == PK_U * 32) {
        pk_u4* d = (pk_u4*)(dst + wb * 36);
        const pk_u4* o = (const pk_u4*)out;
        for (int c = threadIdx.x; c < PK_WORDS / 4; c += 256) __builtin_nontemporal_store(o[c], &d[c]);
    } else {
        unsigned int* d = (unsigned int*)__builtin_assume_aligned(dst + wb * 36, 4);
        for (int c = threadIdx.x; c < nb * 9; c += 256) __builtin_nontemporal_store(out[c], &d[c]);
    }
}

static unsigned pack_grid(long nblocks) { return (unsigned)((nblocks + PK_U * 32 - 1) / (PK_U * 32)); }

/* Launches the pack of nblocks blocks, on the aligned path when src and dst allow it. */
template <bool SRC_BF16>
void launch_pack_q8(const void* src, unsigned char* dst, long nblocks, hipStream_t s) {
    const bool aligned = ((uintptr_t)src & (SRC_BF16 ? 7 : 15)) == 0 && ((uintptr_t)dst & 15) == 0;
    if (aligned)
        hipLaunchKernelGGL((k_quantize_q8<SRC_BF16, true>), dim3(pack_grid(nblocks)), dim3(256), 0, s, src, dst, nblocks);
    else
        hipLaunchKernelGGL((k_quantize_q8<SRC_BF16, false>), dim3(pack_grid(nblocks)), dim3(256), 0, s, src, dst,
                           nblocks);
}

template <bool SRC_BF16>
int launch_quantize(const bmk_launch_t* a) {
    /* buffers: [0] src (fp32 or bf16), [1] dst q8 blocks, [2] params {n} */
    BMK_NEED_BYTES(a, 2, 4, "params");
    const long n = (long)(unsigned int)bmk_pi(a, 2, 0);
    BMK_REQUIRE(n > 0 && n % 32 == 0, "quantize_q8: n=%ld must be a positive multiple of 32", n);
    const long nblocks = n / 32;
    BMK_NEED_BYTES(a, 0, n * (SRC_BF16 ? 2 : 4), "src");
    BMK_NEED_BYTES(a, 1, nblocks * 36, "dst");
    BMK_REQUIRE(((uintptr_t)a->dev[0] & (SRC_BF16 ? 7 : 3)) == 0 && ((uintptr_t)a->dev[1] & 3) == 0,
                "quantize_q8: misaligned src/dst offset");
    launch_pack_q8<SRC_BF16>(a->dev[0], (unsigned char*)a->dev[1], nblocks, a->stream);
    BMK_LAUNCH_CHECK();
    return 0;
}

/* ---- Q4_0 (reference src/baremetal/quant.c:31-52): scale = amax / 7.0f,
 * codes clamp((int)lroundf(p * inv), -8, 7), element 2j in the low nibble
 * of qs[j] and 2j+1 in the high nibble; 20-byte blocks {scale, qs[16]}.
 * Same mapping as the Q8 pack: 8 lanes per block, 4 elements (two bytes of
 * qs) per lane; even lanes join their odd neighbour's two bytes and store
 * one dword. */
__device__ __forceinline__ int q4_round_clamp(float y) {
    if (!(fabsf(y) <= 3.402823466e38f)) return 0; /* NaN / Inf: (int)LONG_MIN == 0 */
    float t = truncf(y);
    if (fabsf(y - t) >= 0.5f) t += copysignf(1.0f, y);
    t = fminf(fmaxf(t, -8.0f), 7.0f);
    return (int)t;
}

template <bool SRC_BF16>
__global__ __launch_bounds__(256) void k_quantize_q4(const void* __restrict__ src, unsigned char* __restrict__ dst,
                                                     long nblocks) {
    const long gt = (long)blockIdx.x * 256 + threadIdx.x;
    const long blk = gt >> 3;
    const int j = threadIdx.x & 7;
    const bool active = blk < nblocks;

    float v[4] = {0.f, 0.f, 0.f, 0.f};
    if (active) load4<SRC_BF16>(src, blk * 32 + 4 * j, v);

    float m = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        float a = fabsf(v[i]);
        m = (a > m) ? a : m;
    }
#pragma unroll
    for (int off = 1; off < 8; off <<= 1) {
        float o = __shfl_xor(m, off, 8);
        m = (o > m) ? o : m;
    }

    const float scale = m / 7.0f;
    unsigned int half = 0u; /* this lane's 4 nibbles: qs bytes 2j and 2j+1 */
    if (scale != 0.0f) {
        const float inv = 1.0f / scale;
#pragma unroll
        for (int i = 0; i < 4; i++) half |= ((unsigned int)q4_round_clamp(v[i] * inv) & 0xFu) << (4 * i);
    }
    const unsigned int other = __shfl_xor(half, 1, 8);
    if (active && (j & 1) == 0) {
        unsigned int* bw = (unsigned int*)__builtin_assume_aligned(dst + blk * 20, 4);
        bw[1 + (j >> 1)] = half | (other << 16);
        if (j == 0) bw[0] = __float_as_uint(scale);
    }
}

template <bool SRC_BF16>
int launch_quantize_q4(const bmk_launch_t* a) {
    /* buffers: [0] src (fp32 or bf16), [1] dst q4 blocks, [2] params {n} */
    BMK_NEED_BYTES(a, 2, 4, "params");
    const long n = (long)(unsigned int)bmk_pi(a, 2, 0);
    BMK_REQUIRE(n > 0 && n % 32 == 0, "quantize_q4: n=%ld must be a positive multiple of 32", n);
    const long nblocks = n / 32;
    BMK_NEED_BYTES(a, 0, n * (SRC_BF16 ? 2 : 4), "src");
    BMK_NEED_BYTES(a, 1, nblocks * 20, "dst");
    BMK_REQUIRE(((uintptr_t)a->dev[0] & (SRC_BF16 ? 7 : 3)) == 0 && ((uintptr_t)a->dev[1] & 3) == 0,
                "quantize_q4: misaligned src/dst offset");
    const unsigned grid = (unsigned)((nblocks * 8 + 255) / 256);
    hipLaunchKernelGGL(k_quantize_q4<SRC_BF16>, dim3(grid), dim3(256), 0, a->stream, (const void*)a->dev[0],
                       (unsigned char*)a->dev[1], nblocks);
    BMK_LAUNCH_CHECK();
    return 0;
}

} // namespace

extern "C" int bmk_launch_quantize_q4(const bmk_launch_t* a) { return launch_quantize_q4<false>(a); }
extern "C" int bmk_launch_quantize_q4_bf16(const bmk_launch_t* a) { return launch_quantize_q4<true>(a); }

/* Engine-side Q4 pack of n bf16 values (the reference's bmt_quantize_q4_bf16). */
extern "C" int q4_pack_bf16(const void* src, unsigned char* dst, long n, hipStream_t s) {
    const long nblocks = n / 32;
    const unsigned grid = (unsigned)((nblocks * 8 + 255) / 256);
    hipLaunchKernelGGL(k_quantize_q4<true>, dim3(grid), dim3(256), 0, s, src, dst, nblocks);
    BMK_LAUNCH_CHECK();
    return 0;
}

/* Engine-side Q4 pack of n fp32 values (as q8_pack_f32). */
extern "C" int q4_pack_f32(const float* src, unsigned char* dst, long n, hipStream_t s) {
    const long nblocks = n / 32;
    const unsigned grid = (unsigned)((nblocks * 8 + 255) / 256);
    hipLaunchKernelGGL(k_quantize_q4<false>, dim3(grid), dim3(256), 0, s, (const void*)src, dst, nblocks);
    BMK_LAUNCH_CHECK();
    return 0;
}

/* Engine-side pack of n bf16 values (the reference's bmt_quantize_q8_bf16;
 * src 8-byte aligned, n a positive multiple of 32). */
extern "C" int q8_pack_bf16(const void* src, unsigned char* dst, long n, hipStream_t s) {
    launch_pack_q8<true>(src, dst, n / 32, s);
    BMK_LAUNCH_CHECK();
    return 0;
}

extern "C" int bmk_launch_quantize_q8(const bmk_launch_t* a) { return launch_quantize<false>(a); }
extern "C" int bmk_launch_quantize_q8_bf16(const bmk_launch_t* a) { return launch_quantize<true>(a); }

/* Engine-side pack of n fp32 values (n a positive multiple of 32, src 4-byte
 * and dst 4-byte aligned; checked by the caller). */
extern "C" int q8_pack_f32(const float* src, unsigned char* dst, long n, hipStream_t s) {
    launch_pack_q8<false>(src, dst, n / 32, s);
    BMK_LAUNCH_CHECK();
    return 0;
}
