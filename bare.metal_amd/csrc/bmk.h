/* SPDX-License-Identifier: MPL-2.0
 *
 * bmk.h — internal interface between the HIP backend (hip_backend.cpp) and
 * the gfx950 kernel files.  Every named kernel is one bmk_desc_t: its name
 * (the string the engine passes to backend_kernel_create), how many buffers
 * it binds, which of them are small parameter blocks that travel by value,
 * which of them it writes, and a launcher that turns the Metal-style
 * dispatch (total threads per axis) into a gfx950 launch of its own shape.
 */
#ifndef BMK_INTERNAL_H
#define BMK_INTERNAL_H

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#define BMK_MAX_BUFFERS 12

typedef struct {
    hipStream_t stream;
    int         n;                         /* buffers bound */
    void*       dev[BMK_MAX_BUFFERS];      /* device address + offset */
    const void* val[BMK_MAX_BUFFERS];      /* host snapshot + offset (by-value buffers only) */
    size_t      bytes[BMK_MAX_BUFFERS];    /* bytes available from the offset to the end */
    int         grid[3];                   /* Metal-style total threads */
    int         tg[3];                     /* Metal-style threadgroup size */
} bmk_launch_t;

/* Returns 0 when the kernel was launched, -1 when the arguments were
 * rejected (nothing launched, error logged). */
typedef int (*bmk_launcher_fn)(const bmk_launch_t* a);

typedef struct {
    const char*     name;
    int             n_buffers;   /* minimum number of bound buffers */
    uint32_t        val_mask;    /* bit i: buffer i is read by value at encode time */
    uint32_t        out_mask;    /* bit i: the kernel may write buffer i */
    bmk_launcher_fn launch;
    uint32_t        dev_mask;    /* bit i (with val_mask): also copied to the device, for kernels that
                                    read a host-validated table from device memory */
} bmk_desc_t;

#ifdef __cplusplus
extern "C" {
#endif
/* Kernel table, terminated by an entry with name == NULL. */
extern const bmk_desc_t bmk_table[];
const bmk_desc_t* bmk_find(const char* name);
void bmk_log(const char* level, const char* file, int line, const char* fmt, ...);
#ifdef __cplusplus
}
#endif

#define BMK_ERR(...)  bmk_log("ERROR", __FILE__, __LINE__, __VA_ARGS__)
#define BMK_WARN(...) bmk_log("WARN", __FILE__, __LINE__, __VA_ARGS__)
#define BMK_INFO(...) bmk_log("INFO", __FILE__, __LINE__, __VA_ARGS__)

/* Read a by-value int/float parameter; the launcher has already checked that
 * buffer i holds at least (k+1)*4 bytes. */
static inline int   bmk_pi(const bmk_launch_t* a, int i, int k) { return ((const int*)a->val[i])[k]; }
static inline float bmk_pf(const bmk_launch_t* a, int i, int k) { return ((const float*)a->val[i])[k]; }

/* Argument checks shared by the launchers. */
#define BMK_REQUIRE(cond, ...) do { if (!(cond)) { BMK_ERR(__VA_ARGS__); return -1; } } while (0)
#define BMK_NEED_BYTES(a, i, nbytes, what) \
    BMK_REQUIRE((a)->bytes[i] >= (size_t)(nbytes), "%s: buffer %d (%s) holds %zu bytes, needs %zu", \
                __func__, i, what, (a)->bytes[i], (size_t)(nbytes))
#define BMK_LAUNCH_CHECK() do { hipError_t e_ = hipGetLastError(); \
    if (e_ != hipSuccess) { BMK_ERR("%s: launch failed: %s", __func__, hipGetErrorString(e_)); return -1; } } while (0)

#endif /* BMK_INTERNAL_H */
