/* noalloc_scratch.cpp -- the device memory behind vq_argmin_noalloc.
 *
 * Compiled as HIP (host + gfx950 device code) and linked into libncmhip.so.
 * `scratch` is a file-scope device array that the code object reserves on
 * every GPU the library runs on, for the lifetime of the process; no call
 * allocates it.  Its name is only a host-side handle: host code never passes
 * it to a kernel.  ncm_noalloc_setup() looks up this device's address of the
 * array once (hipGetSymbolAddress, with the device current) and keeps it per
 * device; every later use goes through ncm_noalloc_scratch(), which returns
 * that address.
 *
 * All calls on one GPU share its array (the library's single stream orders
 * them); calls issued concurrently from several host threads onto that GPU
 * would race on it. */
#include <hip/hip_runtime.h>

#include "noalloc.h"

static __device__ __align__(256) unsigned char scratch[NCM_NOALLOC_SCRATCH_BYTES];

#define NCM_NOALLOC_MAX_DEVICES 64

static void *g_scratch_ptr[NCM_NOALLOC_MAX_DEVICES];
static int g_scratch_err[NCM_NOALLOC_MAX_DEVICES];

extern "C" int ncm_noalloc_setup(int device) {
    if (device < 0 || device >= NCM_NOALLOC_MAX_DEVICES) return (int)hipErrorInvalidDevice;
    if (g_scratch_ptr[device]) return 0;
    void *ptr = nullptr;
    hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr) {
        (void)hipGetLastError();
        g_scratch_err[device] = e != hipSuccess ? (int)e : (int)hipErrorInvalidSymbol;
        return g_scratch_err[device];
    }
    g_scratch_ptr[device] = ptr;
    g_scratch_err[device] = 0;
    return 0;
}

extern "C" void *ncm_noalloc_scratch(int device, int *err) {
    if (device < 0 || device >= NCM_NOALLOC_MAX_DEVICES) {
        if (err) *err = (int)hipErrorInvalidDevice;
        return nullptr;
    }
    if (err) *err = g_scratch_err[device];
    return g_scratch_ptr[device];
}

extern "C" const char *ncm_noalloc_error_string(int err) { return hipGetErrorString((hipError_t)err); }
