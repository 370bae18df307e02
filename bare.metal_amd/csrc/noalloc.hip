/* SPDX-License-Identifier: MPL-2.0
 *
 * noalloc.hip — the device workspace of the engine's no-allocation entry
 * point (bm_forward_noalloc, include/baremetal.h): one file-scope array
 * per GPU, part of the library's code object, so a caller that cannot
 * allocate device memory (serving loops and harnesses that forbid
 * hipMalloc) still gets the prefill's workspace.  Each GPU the
 * library runs on holds BM_NOALLOC_SCRATCH_BYTES until the process ends.
 *
 * In host code `scratch` names a host-side stand-in, not device memory:
 * its device address comes from hipGetSymbolAddress, looked up once per
 * device with that device current and kept per device; only that address
 * is ever handed to kernels or copies.
 */
#include "bmk.h"
#include "baremetal.h"

#include <mutex>

#define BM_NOALLOC_MAX_DEVICES 64

static __device__ __align__(256) unsigned char scratch[BM_NOALLOC_SCRATCH_BYTES];

static void* s_scratch_ptr[BM_NOALLOC_MAX_DEVICES];
static std::mutex s_scratch_mu;

/* Device address of `device`'s workspace (NULL on failure, logged). */
extern "C" void* bmk_noalloc_scratch(int device) {
    if (device < 0 || device >= BM_NOALLOC_MAX_DEVICES) {
        BMK_ERR("no-alloc workspace: device %d outside [0, %d)", device, BM_NOALLOC_MAX_DEVICES);
        return NULL;
    }
    std::lock_guard<std::mutex> lock(s_scratch_mu);
    if (s_scratch_ptr[device]) return s_scratch_ptr[device];
    int cur = -1;
    if (hipGetDevice(&cur) != hipSuccess) {
        BMK_ERR("no-alloc workspace: hipGetDevice failed");
        return NULL;
    }
    if (cur != device && hipSetDevice(device) != hipSuccess) {
        BMK_ERR("no-alloc workspace: hipSetDevice(%d) failed", device);
        return NULL;
    }
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (cur != device) (void)hipSetDevice(cur);
    if (e != hipSuccess || !p) {
        BMK_ERR("no-alloc workspace: hipGetSymbolAddress failed on device %d: %s", device, hipGetErrorString(e));
        return NULL;
    }
    s_scratch_ptr[device] = p;
    return p;
}
