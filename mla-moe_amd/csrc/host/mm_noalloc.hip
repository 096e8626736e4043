/* mm_noalloc.hip -- the MoE FFN entry point that allocates nothing.
 *
 * mm_moe_forward_noalloc_dev runs the same kernels as mm_moe_forward_dev,
 * but its workspace (routing lists, quantised activations, SwiGLU rows,
 * per-route outputs) is a file-scope device array, `scratch`, of a fixed
 * size instead of the context's growable buffer, so the call makes no
 * hipMalloc / hipFree: for callers that cannot allocate (code under HIP
 * graph capture, serving loops, harnesses that forbid it).  The reference
 * has no counterpart.
 *
 * Each device the library runs on holds its own copy of the array until the
 * process ends.  In host code the name `scratch` is only a host-side
 * handle; its device address comes from hipGetSymbolAddress, taken once per
 * device with that device current (mm_noalloc_setup, called by
 * mm_ctx_create) and kept per device.  Every call on a device shares that
 * device's array and leaves its last contents there; no kernel relies on it
 * starting at zero (each workspace region is written before it is read),
 * and calls that overlap on one device (two streams, or two host threads)
 * race on it.
 *
 * This file is compiled by hipcc as host code (plus the device array) and
 * linked into libmlamoe.so with the C11 host objects.
 */
#include <hip/hip_runtime.h>
#include <pthread.h>

extern "C" {
#include "mm_internal.h"
}

static __device__ __align__(256) unsigned char scratch[MM_NOALLOC_SCRATCH_BYTES];

#define MAX_DEVICES 64
static void *g_scratch_ptr[MAX_DEVICES];
static pthread_mutex_t g_lock = PTHREAD_MUTEX_INITIALIZER;

extern "C" int mm_noalloc_setup(mm_ctx *c) {
    if (c->device < 0 || c->device >= MAX_DEVICES)
        return mm_fail(MM_ERR_UNSUPPORTED, "mm_noalloc_setup: device %d >= %d", c->device, MAX_DEVICES);
    pthread_mutex_lock(&g_lock);
    void *p = g_scratch_ptr[c->device];
    hipError_t e = hipSuccess;
    if (!p) {
        e = hipSetDevice(c->device);
        if (e == hipSuccess) e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e == hipSuccess) g_scratch_ptr[c->device] = p;
    }
    pthread_mutex_unlock(&g_lock);
    if (e != hipSuccess) return mm_hip_fail(e, "mm_noalloc_setup: hipGetSymbolAddress(scratch)");
    c->scratch = p;
    c->scratch_bytes = MM_NOALLOC_SCRATCH_BYTES;
    return MM_OK;
}

extern "C" MM_API int mm_moe_forward_noalloc_dev(mm_ctx *c, int layer, int T, const float *xn,
                                                 float *out, const float *logits,
                                                 int32_t *topk_idx, float *topk_w, float *probs,
                                                 unsigned flags) {
    if (!c) return mm_fail(MM_ERR_INVALID, "mm_moe_forward_noalloc_dev: NULL context");
    if (!c->scratch) return mm_fail(MM_ERR_STATE, "mm_moe_forward_noalloc_dev: no scratch on this device");
    /* profiling records are allocated host memory and events: not here */
    if (c->prof_on)
        return mm_fail(MM_ERR_STATE, "mm_moe_forward_noalloc_dev: disable per-kernel profiling first");
    const mm_fixed_ws fx = {(char *)c->scratch, c->scratch_bytes};
    return mm_moe_forward_fixed(c, layer, T, xn, out, logits, topk_idx, topk_w, probs, flags, &fx);
}
