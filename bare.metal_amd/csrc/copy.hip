/* SPDX-License-Identifier: MPL-2.0
 *
 * copy.hip — device-to-device byte copy as a named kernel ("copy_buffer").
 * Used where the engine moves data between buffers on the stream (the
 * reference does such copies on the host through map, e.g.
 * src/baremetal/scheduler.c:1739-1759), and as the plain copy of known size
 * that calibrates HBM byte counters.  16 bytes per lane per step, grid-stride.
 * Also a read-only stream ("stream_read"), the HBM read ceiling.
 */
#include "bmk.h"

namespace {

/* 4 x 16 bytes per lane per step: four loads in flight before the stores */
__global__ __launch_bounds__(256) void k_copy16(const uint4* __restrict__ src, uint4* __restrict__ dst, long n16) {
    const long stride = (long)gridDim.x * 256 * 4;
    long i = (long)blockIdx.x * 256 * 4 + threadIdx.x;
    for (; i + 3 * 256 < n16; i += stride) {
        const uint4 a = src[i], b = src[i + 256], c = src[i + 512], d = src[i + 768];
        dst[i] = a;
        dst[i + 256] = b;
        dst[i + 512] = c;
        dst[i + 768] = d;
    }
    for (int u = 0; u < 4; u++, i += 256)
        if (i < n16) dst[i] = src[i];
}

__global__ __launch_bounds__(256) void k_copy1(const unsigned char* __restrict__ src, unsigned char* __restrict__ dst,
                                               long n) {
    const long i = (long)blockIdx.x * 256 + threadIdx.x;
    if (i < n) dst[i] = src[i];
}

/* Read-only stream: every lane reads 4 x 16 bytes per step (all four in
 * flight before they are combined), grid-stride; each wave writes one xor of
 * what it read so that no load is dead. */
__global__ __launch_bounds__(256) void k_stream_read(const uint4* __restrict__ src, unsigned int* __restrict__ sink,
                                                     long n16) {
    const long stride = (long)gridDim.x * 256 * 4;
    long i = (long)blockIdx.x * 256 * 4 + threadIdx.x;
    unsigned int acc = 0u;
    for (; i + 3 * 256 < n16; i += stride) {
        const uint4 a = src[i], b = src[i + 256], c = src[i + 512], d = src[i + 768];
        acc ^= (a.x ^ a.y ^ a.z ^ a.w) ^ (b.x ^ b.y ^ b.z ^ b.w) ^ (c.x ^ c.y ^ c.z ^ c.w) ^ (d.x ^ d.y ^ d.z ^ d.w);
    }
    for (int u = 0; u < 4; u++, i += 256)
        if (i < n16) acc ^= src[i].x ^ src[i].y ^ src[i].z ^ src[i].w;
    for (int off = 32; off > 0; off >>= 1) acc ^= __shfl_xor(acc, off, 64);
    if ((threadIdx.x & 63) == 0) sink[blockIdx.x * 4 + (threadIdx.x >> 6)] = acc;
}

} // namespace

/* stream_read: the achievable HBM read rate, reported beside the matvec's.
 * buffers {0 src, 1 sink u32 [4 * workgroups], 2 params int64{nbytes, workgroups}};
 * nbytes a multiple of 16, src 16-byte aligned. */
extern "C" int bmk_launch_stream_read(const bmk_launch_t* a) {
    BMK_NEED_BYTES(a, 2, 16, "params");
    long long p[2];
    __builtin_memcpy(p, a->val[2], 16);
    const long long nb = p[0], wg = p[1];
    BMK_REQUIRE(nb > 0 && nb % 16 == 0 && wg > 0 && wg <= 65536, "stream_read: bad params nbytes=%lld workgroups=%lld",
                nb, wg);
    BMK_NEED_BYTES(a, 0, nb, "src");
    BMK_NEED_BYTES(a, 1, wg * 16, "sink");
    BMK_REQUIRE(((uintptr_t)a->dev[0] & 15) == 0 && ((uintptr_t)a->dev[1] & 3) == 0, "stream_read: misaligned buffer");
    hipLaunchKernelGGL(k_stream_read, dim3((unsigned)wg), dim3(256), 0, a->stream, (const uint4*)a->dev[0],
                       (unsigned int*)a->dev[1], (long)(nb / 16));
    BMK_LAUNCH_CHECK();
    return 0;
}

/* buffers {0 src, 1 dst, 2 params int64{nbytes}} */
extern "C" int bmk_launch_copy_buffer(const bmk_launch_t* a) {
    BMK_NEED_BYTES(a, 2, 8, "params");
    long long nb;
    __builtin_memcpy(&nb, a->val[2], 8);
    BMK_REQUIRE(nb >= 0, "copy_buffer: negative size");
    if (nb == 0) return 0;
    BMK_NEED_BYTES(a, 0, nb, "src");
    BMK_NEED_BYTES(a, 1, nb, "dst");
    const unsigned char* s = (const unsigned char*)a->dev[0];
    unsigned char* d = (unsigned char*)a->dev[1];
    const long n16 = ((((uintptr_t)s | (uintptr_t)d) & 15) == 0) ? nb / 16 : 0;
    if (n16 > 0) {
        long blocks = (n16 + 1023) / 1024;
        if (blocks > 256 * 8) blocks = 256 * 8; /* 8 workgroups per CU, grid-stride beyond */
        hipLaunchKernelGGL(k_copy16, dim3((unsigned)blocks), dim3(256), 0, a->stream, (const uint4*)s, (uint4*)d, n16);
        BMK_LAUNCH_CHECK();
    }
    const long tail = nb - n16 * 16;
    if (tail > 0) {
        hipLaunchKernelGGL(k_copy1, dim3((unsigned)((tail + 255) / 256)), dim3(256), 0, a->stream, s + n16 * 16,
                           d + n16 * 16, tail);
        BMK_LAUNCH_CHECK();
    }
    return 0;
}
