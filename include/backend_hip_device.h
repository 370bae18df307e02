/* SPDX-License-Identifier: MPL-2.0
 *
 * backend_hip_device.h — the HIP backend's object layouts.
 *
 * The reference's engine reaches into the backend context for two fields,
 * `supports_bf16` (reference src/baremetal/api.c:13,30) and `library`
 * (reference tools/cli.c:13,98,153,206; tools/run.c:11), through the Metal
 * backend's private header (reference src/backend/metal/device.h:9-43).
 * This header provides the same two fields with the same meaning for the
 * HIP backend: `supports_bf16` is 1 on gfx950 and `library` is non-NULL once
 * the gfx950 kernel table is available, so "is the kernel library loaded"
 * checks in the callers keep working.
 */
#ifndef BMT_BACKEND_HIP_DEVICE_H
#define BMT_BACKEND_HIP_DEVICE_H

#include <stddef.h>
#include <stdint.h>

struct backend_ctx_s {
    void*  device;          /* (intptr_t) HIP device ordinal */
    void*  queue;           /* hipStream_t every encoder records into */
    void*  library;         /* const bmk_desc_t* kernel table (non-NULL when usable) */
    int    supports_bf16;
    size_t allocated_bytes;
    size_t peak_allocated_bytes;

    int    dev_max_threads_per_tg;
    size_t dev_max_threadgroup_mem;
    size_t dev_max_buffer_bytes;
    size_t dev_recommended_working_set;
    int    dev_has_unified_memory;
    int    dev_cu_count;
    int    dev_clock_khz;
    char   dev_name[64];

    double   gpu_busy_ms;
    uint64_t cmd_buffers;

    /* Stream-order bookkeeping for map/unmap: every operation put on the
     * stream takes the next submit epoch; done_epoch is the last epoch known
     * to have completed (after a stream or event synchronisation). */
    uint64_t submit_epoch;
    uint64_t done_epoch;

    /* Recycled hipEvent_t pairs for encoders. */
    void*  event_pool[32];
    int    n_event_pool;
};

struct backend_buffer_s {
    void*   dptr;          /* device memory (hipMalloc) */
    void*   host;          /* pinned host shadow, allocated on first map */
    size_t  size;
    struct backend_ctx_s* ctx;
    int     host_newer;    /* shadow written since the last host->device copy */
    int     dev_newer;     /* a kernel may have written the device copy since the last device->host copy */
    int     fresh;         /* still all-zero since allocation: never bound to a kernel nor unmapped */
    uint64_t last_epoch;   /* last stream epoch that used this buffer */
};

struct backend_kernel_s {
    const void* desc;      /* const bmk_desc_t* */
    struct backend_ctx_s* ctx;
};

struct backend_encoder_s {
    void*   ev_start;      /* hipEvent_t */
    void*   ev_stop;       /* hipEvent_t */
    struct backend_ctx_s* ctx;
    uint64_t commit_epoch;
    int     committed;
    int     n_dispatch;
};

#endif /* BMT_BACKEND_HIP_DEVICE_H */
