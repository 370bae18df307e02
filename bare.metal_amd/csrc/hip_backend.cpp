/* SPDX-License-Identifier: MPL-2.0
 *
 * hip_backend.cpp — the bare.metal backend C ABI (include/backend.h) on HIP
 * for MI355X.  Replaces the Metal implementation (reference
 * src/backend/metal/device.m:16-193, dispatch.m:12-157).
 *
 * Design:
 *   - one context = one HIP device + one non-blocking stream at default
 *     priority; encoders are hipEvent pairs recorded on that stream, so a
 *     Metal command buffer maps to "the work between two events";
 *   - buffers are hipMalloc'd HBM with a pinned host shadow created on the
 *     first map; copies between the two are issued lazily and in stream
 *     order (see include/backend.h for the exact rules);
 *   - kernels are looked up by name in a static table of gfx950 launchers
 *     compiled into this library (the analogue of the metallib +
 *     newFunctionWithName lookup).
 */
#include "bmk.h"
#include "backend.h"
#include "backend_hip_device.h"

#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

/* ------------------------------------------------------------------ */
/* logging (level filter via BAREMETAL_LOG_LEVEL=0..3: error,warn,info,debug) */

static int bmk_log_level(void) {
    static int lvl = -1;
    if (lvl < 0) {
        const char* e = getenv("BAREMETAL_LOG_LEVEL");
        lvl = (e && e[0]) ? atoi(e) : 1;
    }
    return lvl;
}

extern "C" void bmk_log(const char* level, const char* file, int line, const char* fmt, ...) {
    int want = level[0] == 'E' ? 0 : level[0] == 'W' ? 1 : level[0] == 'I' ? 2 : 3;
    if (want > bmk_log_level()) return;
    const char* base = strrchr(file, '/');
    base = base ? base + 1 : file;
    time_t t = time(NULL);
    struct tm tmv;
    localtime_r(&t, &tmv);
    char ts[16];
    strftime(ts, sizeof ts, "%H:%M:%S", &tmv);
    fprintf(stderr, "[%s] %-5s %s:%d: ", ts, level, base, line);
    va_list ap;
    va_start(ap, fmt);
    vfprintf(stderr, fmt, ap);
    va_end(ap);
    fputc('\n', stderr);
}

#define HIP_OK(call, what) hip_ok((call), what, __FILE__, __LINE__)
static bool hip_ok(hipError_t e, const char* what, const char* file, int line) {
    if (e == hipSuccess) return true;
    bmk_log("ERROR", file, line, "%s: %s", what, hipGetErrorString(e));
    return false;
}

static inline hipStream_t ctx_stream(backend_ctx_t* ctx) { return (hipStream_t)ctx->queue; }

static void ctx_sync(backend_ctx_t* ctx) {
    HIP_OK(hipStreamSynchronize(ctx_stream(ctx)), "hipStreamSynchronize");
    ctx->done_epoch = ctx->submit_epoch;
}

/* ------------------------------------------------------------------ */
/* context */

extern "C" backend_ctx_t* backend_create(void) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) {
        (void)hipGetLastError();
        BMK_ERR("No HIP device found");
        return NULL;
    }
    int dev = 0;
    if (!HIP_OK(hipGetDevice(&dev), "hipGetDevice")) return NULL;
    hipDeviceProp_t prop;
    if (!HIP_OK(hipGetDeviceProperties(&prop, dev), "hipGetDeviceProperties")) return NULL;

    backend_ctx_t* ctx = (backend_ctx_t*)calloc(1, sizeof(backend_ctx_t));
    if (!ctx) return NULL;
    hipStream_t s = nullptr;
    if (!HIP_OK(hipStreamCreateWithFlags(&s, hipStreamNonBlocking), "hipStreamCreate")) {
        free(ctx);
        return NULL;
    }
    ctx->device = (void*)(intptr_t)dev;
    ctx->queue = (void*)s;
    ctx->library = (void*)bmk_table;
    ctx->supports_bf16 = 1;
    ctx->dev_max_threads_per_tg = prop.maxThreadsPerBlock;
    ctx->dev_max_threadgroup_mem = prop.sharedMemPerBlock;
    ctx->dev_max_buffer_bytes = prop.totalGlobalMem;
    ctx->dev_recommended_working_set = prop.totalGlobalMem;
    ctx->dev_has_unified_memory = 0;
    ctx->dev_cu_count = prop.multiProcessorCount;
    ctx->dev_clock_khz = prop.clockRate;
    snprintf(ctx->dev_name, sizeof ctx->dev_name, "%s", prop.gcnArchName);
    BMK_INFO("HIP device %d: %s, %d CUs, %zu MiB HBM", dev, prop.gcnArchName,
             prop.multiProcessorCount, (size_t)(prop.totalGlobalMem >> 20));
    return ctx;
}

extern "C" void backend_destroy(backend_ctx_t* ctx) {
    if (!ctx) return;
    if (ctx->queue) {
        ctx_sync(ctx);
        HIP_OK(hipStreamDestroy(ctx_stream(ctx)), "hipStreamDestroy");
    }
    for (int i = 0; i < ctx->n_event_pool; i++)
        HIP_OK(hipEventDestroy((hipEvent_t)ctx->event_pool[i]), "hipEventDestroy");
    free(ctx);
}

extern "C" size_t backend_get_allocated_memory(backend_ctx_t* ctx) {
    return ctx ? ctx->allocated_bytes : 0;
}

extern "C" size_t backend_get_peak_allocated_memory(backend_ctx_t* ctx) {
    return ctx ? ctx->peak_allocated_bytes : 0;
}

extern "C" void backend_get_device_info(backend_ctx_t* ctx, backend_device_info_t* out) {
    if (!ctx || !out) return;
    out->max_threads_per_threadgroup = ctx->dev_max_threads_per_tg;
    out->max_threadgroup_memory = ctx->dev_max_threadgroup_mem;
    out->max_buffer_bytes = ctx->dev_max_buffer_bytes;
    out->recommended_max_working_set = ctx->dev_recommended_working_set;
    out->has_unified_memory = ctx->dev_has_unified_memory;
}

extern "C" double backend_get_gpu_busy_ms(backend_ctx_t* ctx) { return ctx ? ctx->gpu_busy_ms : 0.0; }
extern "C" uint64_t backend_get_command_buffers(backend_ctx_t* ctx) { return ctx ? ctx->cmd_buffers : 0; }
extern "C" void backend_reset_gpu_timing(backend_ctx_t* ctx) {
    if (!ctx) return;
    ctx->gpu_busy_ms = 0.0;
    ctx->cmd_buffers = 0;
}

/* ------------------------------------------------------------------ */
/* buffers */

extern "C" backend_buffer_t* backend_buffer_alloc(backend_ctx_t* ctx, size_t size) {
    if (!ctx || size == 0) return NULL;
    void* d = nullptr;
    if (hipMalloc(&d, size) != hipSuccess) {
        (void)hipGetLastError();
        BMK_ERR("Failed to allocate %zu bytes", size);
        return NULL;
    }
    /* Fresh buffers read as zero, stream-ordered before any later use. */
    if (!HIP_OK(hipMemsetAsync(d, 0, size, ctx_stream(ctx)), "hipMemsetAsync")) {
        (void)hipFree(d);
        return NULL;
    }
    backend_buffer_t* buf = (backend_buffer_t*)calloc(1, sizeof(backend_buffer_t));
    if (!buf) {
        (void)hipFree(d);
        return NULL;
    }
    buf->dptr = d;
    buf->size = size;
    buf->ctx = ctx;
    buf->fresh = 1;
    buf->last_epoch = ++ctx->submit_epoch;
    ctx->allocated_bytes += size;
    if (ctx->allocated_bytes > ctx->peak_allocated_bytes) ctx->peak_allocated_bytes = ctx->allocated_bytes;
    return buf;
}

extern "C" void backend_buffer_free(backend_buffer_t* buf) {
    if (!buf) return;
    backend_ctx_t* ctx = buf->ctx;
    if (ctx && buf->last_epoch > ctx->done_epoch) ctx_sync(ctx);
    if (ctx && ctx->allocated_bytes >= buf->size) ctx->allocated_bytes -= buf->size;
    if (buf->dptr) HIP_OK(hipFree(buf->dptr), "hipFree");
    if (buf->host) HIP_OK(hipHostFree(buf->host), "hipHostFree");
    free(buf);
}

/* Make sure the shadow exists; returns false on allocation failure. */
static bool ensure_shadow(backend_buffer_t* buf) {
    if (buf->host) return true;
    void* h = nullptr;
    if (!HIP_OK(hipHostMalloc(&h, buf->size, hipHostMallocDefault), "hipHostMalloc")) return false;
    buf->host = h;
    if (buf->fresh) {
        memset(h, 0, buf->size); /* same contents as the zero-filled device copy */
        buf->dev_newer = 0;
    } else {
        buf->dev_newer = 1; /* the shadow has never held the device contents */
    }
    return true;
}

/* Bring the shadow up to date with the device copy (waits on the stream). */
static bool shadow_pull(backend_buffer_t* buf) {
    backend_ctx_t* ctx = buf->ctx;
    if (!ensure_shadow(buf)) return false;
    if (buf->last_epoch > ctx->done_epoch) ctx_sync(ctx);
    if (buf->dev_newer && !buf->host_newer) {
        if (!HIP_OK(hipMemcpyAsync(buf->host, buf->dptr, buf->size, hipMemcpyDeviceToHost, ctx_stream(ctx)),
                    "hipMemcpy D2H"))
            return false;
        buf->last_epoch = ++ctx->submit_epoch;
        ctx_sync(ctx);
        buf->dev_newer = 0;
    }
    return true;
}

extern "C" void* backend_buffer_map(backend_buffer_t* buf) {
    if (!buf || !buf->dptr) return NULL;
    if (!shadow_pull(buf)) return NULL;
    return buf->host;
}

extern "C" void backend_buffer_unmap(backend_buffer_t* buf) {
    if (!buf || !buf->host) return;
    buf->host_newer = 1;
    buf->fresh = 0;
}

extern "C" size_t backend_buffer_size(backend_buffer_t* buf) { return buf ? buf->size : 0; }

/* Issue the host->device copy of a shadow the host has written (stream order). */
static bool shadow_push(backend_buffer_t* buf) {
    if (!buf->host_newer) return true;
    backend_ctx_t* ctx = buf->ctx;
    if (!HIP_OK(hipMemcpyAsync(buf->dptr, buf->host, buf->size, hipMemcpyHostToDevice, ctx_stream(ctx)),
                "hipMemcpy H2D"))
        return false;
    buf->host_newer = 0;
    buf->dev_newer = 0;
    buf->last_epoch = ++ctx->submit_epoch;
    return true;
}

/* ------------------------------------------------------------------ */
/* kernels */

extern "C" const bmk_desc_t* bmk_find(const char* name) {
    if (!name) return NULL;
    for (const bmk_desc_t* d = bmk_table; d->name; d++)
        if (strcmp(d->name, name) == 0) return d;
    return NULL;
}

extern "C" backend_kernel_t* backend_kernel_create(backend_ctx_t* ctx, const char* name) {
    if (!ctx || !ctx->library || !name) return NULL;
    const bmk_desc_t* d = bmk_find(name);
    if (!d) {
        BMK_ERR("Kernel not found: %s", name);
        return NULL;
    }
    backend_kernel_t* k = (backend_kernel_t*)calloc(1, sizeof(backend_kernel_t));
    if (!k) return NULL;
    k->desc = d;
    k->ctx = ctx;
    BMK_INFO("Kernel resolved: %s", name);
    return k;
}

extern "C" void backend_kernel_destroy(backend_kernel_t* kernel) { free(kernel); }

/* ------------------------------------------------------------------ */
/* encoders */

static hipEvent_t event_get(backend_ctx_t* ctx) {
    if (ctx->n_event_pool > 0) return (hipEvent_t)ctx->event_pool[--ctx->n_event_pool];
    hipEvent_t e = nullptr;
    if (!HIP_OK(hipEventCreate(&e), "hipEventCreate")) return nullptr;
    return e;
}

static void event_put(backend_ctx_t* ctx, hipEvent_t e) {
    if (!e) return;
    if (ctx->n_event_pool < (int)(sizeof ctx->event_pool / sizeof ctx->event_pool[0]))
        ctx->event_pool[ctx->n_event_pool++] = (void*)e;
    else
        HIP_OK(hipEventDestroy(e), "hipEventDestroy");
}

extern "C" backend_encoder_t* backend_encode_begin(backend_ctx_t* ctx) {
    if (!ctx) return NULL;
    backend_encoder_t* e = (backend_encoder_t*)calloc(1, sizeof(backend_encoder_t));
    if (!e) return NULL;
    e->ctx = ctx;
    hipEvent_t a = event_get(ctx), b = event_get(ctx);
    if (!a || !b) {
        event_put(ctx, a);
        event_put(ctx, b);
        free(e);
        return NULL;
    }
    e->ev_start = (void*)a;
    e->ev_stop = (void*)b;
    HIP_OK(hipEventRecord(a, ctx_stream(ctx)), "hipEventRecord");
    return e;
}

extern "C" int backend_encode_dispatch(backend_encoder_t* enc, backend_kernel_t* kernel, backend_buffer_t* buffers[],
                                       size_t offsets[], int num_buffers, int grid_x, int grid_y, int grid_z,
                                       int tg_x, int tg_y, int tg_z) {
    if (!enc || !kernel || !buffers || enc->committed) return -1;
    const bmk_desc_t* d = (const bmk_desc_t*)kernel->desc;
    backend_ctx_t* ctx = enc->ctx;
    if (num_buffers < d->n_buffers || num_buffers > BMK_MAX_BUFFERS) {
        BMK_ERR("%s: %d buffers bound, kernel needs %d (max %d)", d->name, num_buffers, d->n_buffers,
                BMK_MAX_BUFFERS);
        return -1;
    }
    if (grid_x < 0 || grid_y < 0 || grid_z < 0 || tg_x <= 0 || tg_y <= 0 || tg_z <= 0) {
        BMK_ERR("%s: bad dispatch geometry", d->name);
        return -1;
    }
    bmk_launch_t a;
    memset(&a, 0, sizeof a);
    a.stream = ctx_stream(ctx);
    a.n = num_buffers;
    a.grid[0] = grid_x; a.grid[1] = grid_y; a.grid[2] = grid_z;
    a.tg[0] = tg_x; a.tg[1] = tg_y; a.tg[2] = tg_z;
    for (int i = 0; i < num_buffers; i++) {
        backend_buffer_t* b = buffers[i];
        size_t off = offsets ? offsets[i] : 0;
        if (!b || !b->dptr) {
            BMK_ERR("%s: buffer %d is NULL", d->name, i);
            return -1;
        }
        if (off > b->size) {
            BMK_ERR("%s: buffer %d offset %zu beyond size %zu", d->name, i, off, b->size);
            return -1;
        }
        a.bytes[i] = b->size - off;
        if (d->val_mask & (1u << i)) {
            /* parameter block: snapshot the host view now */
            if (!b->host || (b->dev_newer && !b->host_newer)) {
                if (!shadow_pull(b)) return -1;
            }
            a.val[i] = (const char*)b->host + off;
            if ((d->dev_mask & (1u << i)) && !shadow_push(b)) return -1;
        } else {
            if (!shadow_push(b)) return -1;
        }
        a.dev[i] = (char*)b->dptr + off;
    }
    if (d->launch(&a) != 0) return -1;
    uint64_t ep = ++ctx->submit_epoch;
    for (int i = 0; i < num_buffers; i++) {
        buffers[i]->last_epoch = ep;
        buffers[i]->fresh = 0;
        if (d->out_mask & (1u << i)) buffers[i]->dev_newer = 1;
    }
    enc->n_dispatch++;
    return 0;
}

extern "C" void backend_encode_commit(backend_encoder_t* enc) {
    if (!enc || enc->committed) return;
    HIP_OK(hipEventRecord((hipEvent_t)enc->ev_stop, ctx_stream(enc->ctx)), "hipEventRecord");
    enc->commit_epoch = enc->ctx->submit_epoch;
    enc->committed = 1;
}

extern "C" double backend_encode_wait_timed(backend_encoder_t* enc) {
    if (!enc) return 0.0;
    backend_ctx_t* ctx = enc->ctx;
    if (!enc->committed) backend_encode_commit(enc);
    float ms = 0.0f;
    hipEvent_t a = (hipEvent_t)enc->ev_start, b = (hipEvent_t)enc->ev_stop;
    if (HIP_OK(hipEventSynchronize(b), "hipEventSynchronize")) {
        if (enc->commit_epoch > ctx->done_epoch) ctx->done_epoch = enc->commit_epoch;
        if (hipEventElapsedTime(&ms, a, b) != hipSuccess) {
            (void)hipGetLastError();
            ms = 0.0f;
        }
    }
    ctx->gpu_busy_ms += ms;
    ctx->cmd_buffers += 1;
    event_put(ctx, a);
    event_put(ctx, b);
    free(enc);
    return (double)ms;
}

extern "C" void backend_encode_wait(backend_encoder_t* enc) { (void)backend_encode_wait_timed(enc); }

extern "C" int backend_kernel_dispatch(backend_ctx_t* ctx, backend_kernel_t* kernel, backend_buffer_t* buffers[],
                                       size_t offsets[], int num_buffers, int grid_x, int grid_y, int grid_z,
                                       int tg_x, int tg_y, int tg_z) {
    if (!ctx || !kernel || !buffers) return -1;
    backend_encoder_t* e = backend_encode_begin(ctx);
    if (!e) return -1;
    int rc = backend_encode_dispatch(e, kernel, buffers, offsets, num_buffers, grid_x, grid_y, grid_z, tg_x, tg_y,
                                     tg_z);
    backend_encode_commit(e);
    backend_encode_wait(e);
    return rc;
}

extern "C" void backend_synchronize(backend_ctx_t* ctx) {
    if (ctx) ctx_sync(ctx);
}
