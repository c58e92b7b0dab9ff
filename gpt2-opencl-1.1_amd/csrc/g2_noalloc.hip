/*
 * g2_noalloc.hip -- device scratch of the allocation-free entry point
 * g2_attn_1q_noalloc (g2hip.h).
 *
 * Compiled by hipcc as an ordinary HIP translation unit (host and device
 * code), so the HIP runtime registers this file's device code object and
 * the symbol `scratch` below can be resolved with hipGetSymbolAddress.  The
 * kernels that use it are the library's own single-query attention kernels
 * (g2k_attn_part / g2k_attn_merge in the module-loaded code object); they
 * take the scratch address as an argument, exactly as they take the
 * library-allocated partials buffer in g2_attn_1q.
 *
 * The array lives for the life of the process on every GPU the library
 * runs on.  In host code its name is a host-side stand-in, never a device
 * address: every use goes through the per-device pointer resolved once by
 * g2i_noalloc_setup (called from g2_init with the device current).
 */
#include <hip/hip_runtime.h>

#include "g2_internal.h"

/* Chunk partials of one single-query attention call: (max, sum, o[64]) for
 * each of at most 64 heads x G2_ATTN_MAX_CHUNKS key chunks (270 KB). */
static __device__ __align__(256) float scratch[G2_NOALLOC_SCRATCH_FLOATS];

#define G2_NOALLOC_MAX_DEVICES 64
static void *g_scratch[G2_NOALLOC_MAX_DEVICES];

extern "C" int g2i_noalloc_setup(int device)
{
    if (device < 0 || device >= G2_NOALLOC_MAX_DEVICES)
        return g2i_err(G2_E_ARG, "device %d beyond the %d devices of the static scratch table", device,
                       G2_NOALLOC_MAX_DEVICES);
    if (g_scratch[device]) return G2_OK;
    void *ptr = NULL;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr) {
        (void)hipGetLastError();
        return g2i_err(G2_E_HIP, "hipGetSymbolAddress(scratch): HIP error %d (%s)", (int)e, hipGetErrorString(e));
    }
    g_scratch[device] = ptr;
    return G2_OK;
}

extern "C" float *g2i_noalloc_scratch(int device)
{
    if (device < 0 || device >= G2_NOALLOC_MAX_DEVICES) return NULL;
    return (float *)g_scratch[device];
}
