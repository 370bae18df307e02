/* SPDX-License-Identifier: MPL-2.0
 *
 * backend.h — the bare.metal backend C ABI, implemented for AMD Instinct
 * MI355X (gfx950) by libbaremetal_hip.so.
 *
 * This is the drop-in boundary: the declarations below are the same 22
 * functions and the same device-info struct as the reference's Metal backend
 * interface (reference: src/backend/backend.h:12-67).  The engine above it
 * (scheduler, session, registry) calls only these functions, so the HIP
 * library replaces src/backend/metal/{device.m,dispatch.m} without any change
 * to the callers' code.
 *
 * Semantics that the HIP implementation keeps from the Metal one:
 *   - kernels are resolved by name (reference dispatch.m:16-21) and NULL is
 *     returned, with a logged error, for an unknown name;
 *   - buffers bind by index with optional byte offsets (NULL = all zero)
 *     (reference dispatch.m:117-120);
 *   - grid_* is the TOTAL thread count per axis (Metal dispatchThreads), not a
 *     block count; it need not be a multiple of tg_* (reference
 *     dispatch.m:121-122);
 *   - backend_encode_wait / backend_encode_wait_timed free the encoder
 *     (reference dispatch.m:150-155);
 *   - *_free / *_destroy accept NULL (reference device.m:144-159,182-191).
 * Semantics that differ because MI355X memory is discrete HBM, not unified:
 *   - backend_buffer_map returns a host shadow of the device buffer.  If a
 *     kernel may have written the buffer since the last map, map first waits
 *     for the stream and copies device -> host.  backend_buffer_unmap marks
 *     the shadow as newer than the device copy; the host -> device copy is
 *     issued, in stream order, before the next kernel that binds the buffer.
 *   - Small parameter buffers are read from their host shadow when the
 *     dispatch is encoded and travel as kernel arguments (a snapshot).  The
 *     reference's scheduler writes each parameter buffer before encoding the
 *     node and does not rewrite it before the encoder is waited on
 *     (reference scheduler.c:794-833), so the snapshot sees the same values
 *     the Metal kernel would read.
 *   - has_unified_memory is reported as 0.
 */
#ifndef BMT_BACKEND_H
#define BMT_BACKEND_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct backend_ctx_s     backend_ctx_t;
typedef struct backend_buffer_s  backend_buffer_t;
typedef struct backend_kernel_s  backend_kernel_t;
typedef struct backend_encoder_s backend_encoder_t;

/* reference backend.h:17-20 */
backend_ctx_t*    backend_create(void);
void              backend_destroy(backend_ctx_t* ctx);
size_t            backend_get_allocated_memory(backend_ctx_t* ctx);
size_t            backend_get_peak_allocated_memory(backend_ctx_t* ctx);

/* reference backend.h:22-30 */
typedef struct {
    int    max_threads_per_threadgroup;
    size_t max_threadgroup_memory;
    size_t max_buffer_bytes;
    size_t recommended_max_working_set;
    int    has_unified_memory;
} backend_device_info_t;

void              backend_get_device_info(backend_ctx_t* ctx, backend_device_info_t* out);

/* reference backend.h:32-38: GPU busy time is the sum of the hipEvent
 * intervals of every waited encoder. */
double            backend_get_gpu_busy_ms(backend_ctx_t* ctx);
uint64_t          backend_get_command_buffers(backend_ctx_t* ctx);
void              backend_reset_gpu_timing(backend_ctx_t* ctx);
double            backend_encode_wait_timed(backend_encoder_t* enc);

/* reference backend.h:40-44 */
backend_buffer_t* backend_buffer_alloc(backend_ctx_t* ctx, size_t size);
void              backend_buffer_free(backend_buffer_t* buf);
void*             backend_buffer_map(backend_buffer_t* buf);
void              backend_buffer_unmap(backend_buffer_t* buf);
size_t            backend_buffer_size(backend_buffer_t* buf);

/* reference backend.h:46-47 */
backend_kernel_t* backend_kernel_create(backend_ctx_t* ctx, const char* name);
void              backend_kernel_destroy(backend_kernel_t* kernel);

/* reference backend.h:49-56: one dispatch in its own encoder, waited on. */
int               backend_kernel_dispatch(backend_ctx_t* ctx,
                       backend_kernel_t* kernel,
                       backend_buffer_t* buffers[],
                       size_t offsets[],
                       int num_buffers,
                       int grid_x, int grid_y, int grid_z,
                       int tg_x,  int tg_y,  int tg_z);
void              backend_synchronize(backend_ctx_t* ctx);

/* reference backend.h:58-67 */
backend_encoder_t* backend_encode_begin(backend_ctx_t* ctx);
int               backend_encode_dispatch(backend_encoder_t* enc,
                       backend_kernel_t* kernel,
                       backend_buffer_t* buffers[],
                       size_t offsets[],
                       int num_buffers,
                       int grid_x, int grid_y, int grid_z,
                       int tg_x,  int tg_y,  int tg_z);
void              backend_encode_commit(backend_encoder_t* enc);
void              backend_encode_wait(backend_encoder_t* enc);

#ifdef __cplusplus
}
#endif

#endif /* BMT_BACKEND_H */
