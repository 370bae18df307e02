/* SPDX-License-Identifier: MPL-2.0
 *
 * q8_common.h — device helpers shared by the quantized kernels: one 36-byte
 * Q8_0 block {f32 scale; int8 q[32]} (reference src/baremetal/quant.h:17-32)
 * read with two dwordx4 loads and one dword load, one 20-byte Q4_0 block
 * (quant.h:34-42) read with a dword and a dwordx4 load, and their dot
 * products with 32 fp32 activations held in registers.
 */
#ifndef BMK_Q8_COMMON_H
#define BMK_Q8_COMMON_H

#include <hip/hip_runtime.h>

namespace bmk {

struct Blk {
    float s;
    uint4 q0, q1;
};

__device__ __forceinline__ Blk load_block(const unsigned char* p) {
    Blk b;
    unsigned char raw[36];
    __builtin_memcpy(raw, __builtin_assume_aligned(p, 4), 36);
    __builtin_memcpy(&b.s, raw, 4);
    __builtin_memcpy(&b.q0, raw + 4, 16);
    __builtin_memcpy(&b.q1, raw + 20, 16);
    return b;
}

/* fp32 -> bf16 bits, round to nearest even (v_cvt_pk_bf16_f32) */
__device__ __forceinline__ unsigned short bf16_bits(float v) {
    typedef float f32x2_t __attribute__((ext_vector_type(2)));
    typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
    const f32x2_t f = {v, 0.0f};
    const bf16x2_t r = __builtin_convertvector(f, bf16x2_t);
    unsigned int u;
    __builtin_memcpy(&u, &r, 4);
    return (unsigned short)(u & 0xffffu);
}

/* int8 k (0..3) of a packed dword, exactly as fp32 */
__device__ __forceinline__ float q8_byte(unsigned int w, int k) { return (float)(signed char)((w >> (8 * k)) & 0xffu); }

__device__ __forceinline__ float dot4(unsigned int w, const float* x) {
    float a = x[0] * (float)(signed char)(w & 0xffu);
    a = fmaf(x[1], (float)(signed char)((w >> 8) & 0xffu), a);
    a = fmaf(x[2], (float)(signed char)((w >> 16) & 0xffu), a);
    a = fmaf(x[3], (float)(signed char)(w >> 24), a);
    return a;
}

__device__ __forceinline__ float block_dot(const Blk& b, const float* xs) {
    float s0 = dot4(b.q0.x, xs + 0) + dot4(b.q0.y, xs + 4);
    float s1 = dot4(b.q0.z, xs + 8) + dot4(b.q0.w, xs + 12);
    float s2 = dot4(b.q1.x, xs + 16) + dot4(b.q1.y, xs + 20);
    float s3 = dot4(b.q1.z, xs + 24) + dot4(b.q1.w, xs + 28);
    return ((s0 + s1) + (s2 + s3)) * b.s;
}


/* ---- Q4_0 blocks: 20 bytes {f32 scale; u8 qs[16]} (reference
 * src/baremetal/quant.h:34-42); element 2j is the low nibble of qs[j],
 * element 2j+1 the high nibble, each a two's-complement 4-bit code. */
struct Blk4 {
    float s;
    uint4 q;
};

__device__ __forceinline__ Blk4 load_block4(const unsigned char* p) {
    Blk4 b;
    __builtin_memcpy(&b.s, __builtin_assume_aligned(p, 4), 4);
    __builtin_memcpy(&b.q, __builtin_assume_aligned(p + 4, 4), 16);
    return b;
}

__device__ __forceinline__ Blk4 zero_block4() {
    Blk4 b;
    b.s = 0.0f;
    b.q = make_uint4(0, 0, 0, 0);
    return b;
}

/* code k (0..7) of a dword of packed nibbles, exactly as fp32 */
__device__ __forceinline__ float q4_code(unsigned int w, int k) { return (float)((int)(w << (28 - 4 * k)) >> 28); }

__device__ __forceinline__ float dot8_q4(unsigned int w, const float* x) {
    float a = x[0] * q4_code(w, 0);
#pragma unroll
    for (int k = 1; k < 8; k++) a = fmaf(x[k], q4_code(w, k), a);
    return a;
}

__device__ __forceinline__ float block_dot(const Blk4& b, const float* xs) {
    const float s0 = dot8_q4(b.q.x, xs + 0) + dot8_q4(b.q.y, xs + 8);
    const float s1 = dot8_q4(b.q.z, xs + 16) + dot8_q4(b.q.w, xs + 24);
    return (s0 + s1) * b.s;
}

/* Block formats of the quantized kernels: bytes per 32-weight block and the
 * register form of one block. */
enum { QF_Q8 = 0, QF_Q4 = 1 };
template <int QF> struct QFmt;
template <> struct QFmt<QF_Q8> {
    static constexpr int BYTES = 36;
    typedef Blk Block;
    static __device__ __forceinline__ Blk load(const unsigned char* p) { return load_block(p); }
    static __device__ __forceinline__ Blk zero();
};
template <> struct QFmt<QF_Q4> {
    static constexpr int BYTES = 20;
    typedef Blk4 Block;
    static __device__ __forceinline__ Blk4 load(const unsigned char* p) { return load_block4(p); }
    static __device__ __forceinline__ Blk4 zero() { return zero_block4(); }
};

__device__ __forceinline__ Blk zero_block() {
    Blk b;
    b.s = 0.0f;
    b.q0 = make_uint4(0, 0, 0, 0);
    b.q1 = make_uint4(0, 0, 0, 0);
    return b;
}

__device__ __forceinline__ Blk QFmt<QF_Q8>::zero() { return zero_block(); }

/* Sum over the 64 lanes of a wave (xor butterfly; every lane gets the sum). */
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
    return v;
}

/* Index of A[row][col] in MFMA fragment order, the activation layout the
 * prefill GEMMs load (q8_gemm.hip's gemm_tile_frag, pf_gemm.hip): 32-row
 * blocks rb and 64-column steps ks of four 16-deep fragments of 512 values;
 * fragment (rb, ks, s) starts at ((rb * nks + ks) * 4 + s) * 512 and lane
 * l's eight values at + 8 l hold A[32 rb + l % 32][64 ks + 32 (l / 32) +
 * 8 s + j], j < 8 (nks = ceil(K / 64)).  Eight consecutive columns from a
 * multiple of 8 are eight consecutive values. */
__host__ __device__ __forceinline__ size_t frag_index(int row, int col, int nks) {
    const int rb = row >> 5, lr = row & 31, ks = col >> 6, h = (col >> 5) & 1, s = (col >> 3) & 3;
    return ((size_t)(rb * nks + ks) * 4 + s) * 512 + 8 * (lr + 32 * h) + (col & 7);
}

/* silu(g) * u, the SwiGLU product (reference forward.metal:1179-1190) */
__device__ __forceinline__ float silu_mul(float g, float u) { return (g / (1.0f + expf(-g))) * u; }

} // namespace bmk

#endif
