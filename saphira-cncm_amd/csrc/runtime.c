/* runtime.c -- HIP runtime shim of libncmhip: device selection, the single
 * library stream, the embedded gfx950 code objects, kernel launch, error
 * policy, and the ncm.h memory substrate (Tensor, arenas, mem_* copies) that
 * the reference implements in src/tensor.c. */
#include "internal.h"
#include "noalloc.h"

#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

/* ---- embedded code objects (blobs.S) ---- */
extern const unsigned char ncm_co_gemm[], ncm_co_vq[], ncm_co_ops[], ncm_co_train[], ncm_co_sample[], ncm_co_ncp[];
static const unsigned char *const co_blobs[] = {ncm_co_gemm, ncm_co_vq, ncm_co_ops, ncm_co_train, ncm_co_sample,
                                                ncm_co_ncp};
#define N_MODULES (int)(sizeof(co_blobs) / sizeof(co_blobs[0]))

static int g_state = 0; /* 0 = not initialised, 1 = ready, <0 = failed */
static int g_device = 0;
static int g_cus = 0;
static hipStream_t g_stream = NULL;
static hipModule_t g_mod[N_MODULES];
static int g_err_mode = NCM_ERR_EXIT;
static int g_err_code = 0;
static char g_err_msg[512];

int ncm_fail(int code, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err_msg, sizeof(g_err_msg), fmt, ap);
    va_end(ap);
    g_err_code = code;
    if (g_err_mode == NCM_ERR_EXIT) {
        fprintf(stderr, "ncmhip: %s\n", g_err_msg);
        exit(1);
    }
    return code;
}

void ncm_hip_set_error_mode(int mode) { g_err_mode = mode; }

int ncm_hip_last_error(char *buf, size_t cap) {
    int c = g_err_code;
    if (buf && cap) {
        strncpy(buf, c ? g_err_msg : "", cap - 1);
        buf[cap - 1] = 0;
    }
    g_err_code = 0;
    return c;
}

int ncm_hip_init(int device) {
    if (g_state == 1) return 0;
    if (g_state < 0) return ncm_fail(NCM_E_INIT, "runtime initialisation failed earlier");
    g_state = -1;
    int n = 0;
    HIP_TRY(hipGetDeviceCount(&n));
    if (n <= 0) return ncm_fail(NCM_E_INIT, "no HIP device visible");
    if (device < 0 || device >= n)
        return ncm_fail(NCM_E_INIT, "device %d out of range (%d devices)", device, n);
    HIP_TRY(hipSetDevice(device));
    /* the fixed device array behind the allocation-free entry points: its
     * address on this device, looked up once with the device current (a
     * failure is reported by those entry points, not here) */
    (void)ncm_noalloc_setup(device);
    hipDeviceProp_t prop;
    HIP_TRY(hipGetDeviceProperties(&prop, device));
    if (strncmp(prop.gcnArchName, "gfx950", 6) != 0)
        return ncm_fail(NCM_E_INIT, "device %d is %s; this library is built for gfx950 only",
                        device, prop.gcnArchName);
    g_cus = prop.multiProcessorCount;
    HIP_TRY(hipStreamCreateWithFlags(&g_stream, hipStreamNonBlocking));
    for (int i = 0; i < N_MODULES; i++) HIP_TRY(hipModuleLoadData(&g_mod[i], co_blobs[i]));
    g_device = device;
    g_state = 1;
    return 0;
}

int ncm_ready(void) {
    if (g_state == 1) return 0;
    const char *e = getenv("NCM_DEVICE");
    return ncm_hip_init(e ? atoi(e) : 0);
}

hipStream_t ncm_stream(void) { return g_stream; }
int ncm_device(void) { return g_device; }
void *ncm_hip_stream(void) { return ncm_ready() ? NULL : (void *)g_stream; }

void ncm_hip_sync(void) {
    if (ncm_ready()) return;
    hipError_t e = hipStreamSynchronize(g_stream);
    if (e != hipSuccess) ncm_fail(NCM_E_HIP, "stream synchronize: %s", hipGetErrorString(e));
}

/* ---- kernel lookup + launch ---- */
typedef struct {
    char name[64];
    hipFunction_t f;
} KEnt;
static KEnt g_kern[256];
static int g_nkern = 0;

hipFunction_t ncm_kernel(const char *name) {
    for (int i = 0; i < g_nkern; i++)
        if (strcmp(g_kern[i].name, name) == 0) return g_kern[i].f;
    if (ncm_ready()) return NULL;
    for (int m = 0; m < N_MODULES; m++) {
        hipFunction_t f;
        if (hipModuleGetFunction(&f, g_mod[m], name) == hipSuccess) {
            if (g_nkern < (int)(sizeof(g_kern) / sizeof(g_kern[0]))) {
                strncpy(g_kern[g_nkern].name, name, sizeof(g_kern[0].name) - 1);
                g_kern[g_nkern].f = f;
                g_nkern++;
            }
            return f;
        }
    }
    (void)hipGetLastError();
    ncm_fail(NCM_E_INIT, "kernel %s not found in the embedded code objects", name);
    return NULL;
}

int ncm_launch(hipFunction_t f, unsigned gx, unsigned gy, unsigned gz, unsigned block,
               void **args) {
    if (!f) return NCM_E_INIT;
    if (gx == 0 || gy == 0 || gz == 0) return 0;
    HIP_TRY(hipModuleLaunchKernel(f, gx, gy, gz, block, 1, 1, 0, g_stream, args, NULL));
    return 0;
}

int ncm_launch_named(const char *name, unsigned gx, unsigned gy, unsigned gz, unsigned block,
                     void **args) {
    hipFunction_t f = ncm_kernel(name);
    if (!f) return NCM_E_INIT;
    return ncm_launch(f, gx, gy, gz, block, args);
}

/* ---- workspaces ---- */
static void *g_ws[WS_COUNT];
static size_t g_ws_size[WS_COUNT];

void *ncm_workspace(int slot, size_t bytes) {
    if (bytes <= g_ws_size[slot]) return g_ws[slot];
    if (ncm_ready()) return NULL;
    if (g_ws[slot]) {
        hipError_t e = hipStreamSynchronize(g_stream);
        if (e != hipSuccess) {
            ncm_fail(NCM_E_HIP, "workspace grow sync: %s", hipGetErrorString(e));
            return NULL;
        }
        (void)hipFree(g_ws[slot]);
        g_ws[slot] = NULL;
        g_ws_size[slot] = 0;
    }
    size_t sz = bytes < (1u << 20) ? (1u << 20) : bytes;
    sz = (sz + 0xFFFFF) & ~(size_t)0xFFFFF;
    void *p = NULL;
    hipError_t e = hipMalloc(&p, sz);
    if (e != hipSuccess) {
        ncm_fail(NCM_E_OOM, "workspace of %zu bytes: %s", sz, hipGetErrorString(e));
        return NULL;
    }
    g_ws[slot] = p;
    g_ws_size[slot] = sz;
    return p;
}

int ncm_cu_count(void) { return g_cus > 0 ? g_cus : 1; }

/* ---- plain device allocation ---- */
/* Test hook: after this many more successful allocations, ncm_hip_malloc
 * fails as if the device were out of memory (< 0: never). */
static long g_alloc_fail_after = -1;

void ncm_hip_fail_alloc_after(long n) { g_alloc_fail_after = n; }

void *ncm_hip_malloc(size_t bytes) {
    if (ncm_ready()) return NULL;
    if (g_alloc_fail_after == 0) {
        ncm_fail(NCM_E_OOM, "hipMalloc(%zu): failure injected by ncm_hip_fail_alloc_after", bytes);
        return NULL;
    }
    if (g_alloc_fail_after > 0) g_alloc_fail_after--;
    void *p = NULL;
    hipError_t e = hipMalloc(&p, bytes ? bytes : 16);
    if (e != hipSuccess) {
        ncm_fail(NCM_E_OOM, "hipMalloc(%zu): %s", bytes, hipGetErrorString(e));
        return NULL;
    }
    return p;
}

void ncm_hip_free(void *p) {
    if (!p || ncm_ready()) return;
    /* queued kernels may still read p */
    (void)hipStreamSynchronize(g_stream);
    (void)hipFree(p);
}

/* ---- Tensor (tensor.c:15-62) ---- */
int64_t tensor_numel(int ndim, const int64_t *shape) {
    int64_t n = 1;
    for (int i = 0; i < ndim; i++) n *= shape[i];
    return n;
}

Tensor *tensor_alloc(int ndim, const int64_t *shape) {
    if (ndim < 0 || ndim > NCM_MAX_DIMS) {
        ncm_fail(NCM_E_ARG, "tensor_alloc: ndim %d", ndim);
        return NULL;
    }
    Tensor *t = (Tensor *)calloc(1, sizeof(Tensor));
    if (!t) {
        ncm_fail(NCM_E_OOM, "oom tensor");
        return NULL;
    }
    t->ndim = ndim;
    for (int i = 0; i < ndim; i++) t->shape[i] = shape[i];
    t->n = tensor_numel(ndim, shape);
    t->data = (float *)ncm_hip_malloc((size_t)t->n * sizeof(float));
    if (!t->data) {
        free(t);
        return NULL;
    }
    return t;
}

void tensor_free(Tensor *t) {
    if (!t) return;
    ncm_hip_free(t->data);
    free(t);
}

void mem_d2h(void *h, const void *d, size_t n) {
    if (ncm_ready() || n == 0) return;
    hipError_t e = hipMemcpyAsync(h, d, n, hipMemcpyDeviceToHost, g_stream);
    if (e == hipSuccess) e = hipStreamSynchronize(g_stream);
    if (e != hipSuccess) ncm_fail(NCM_E_HIP, "mem_d2h(%zu): %s", n, hipGetErrorString(e));
}

void mem_h2d(void *d, const void *h, size_t n) {
    if (ncm_ready() || n == 0) return;
    hipError_t e = hipMemcpyAsync(d, h, n, hipMemcpyHostToDevice, g_stream);
    if (e == hipSuccess) e = hipStreamSynchronize(g_stream);
    if (e != hipSuccess) ncm_fail(NCM_E_HIP, "mem_h2d(%zu): %s", n, hipGetErrorString(e));
}

/* Small host-to-device uploads (token ids, targets) without a host
 * synchronisation: the bytes are copied into one of a ring of pinned staging
 * slots and sent by an asynchronous copy on the library stream; a slot is
 * reused only once the event recorded behind its last copy has completed.
 * Larger uploads, or a device other than the one the ring was made on, take
 * mem_h2d. */
#define H2D_SLOTS 8
#define H2D_SLOT_BYTES ((size_t)256 << 10)
static unsigned char *g_h2d_pin = NULL;
static hipEvent_t g_h2d_ev[H2D_SLOTS];
static int g_h2d_used[H2D_SLOTS], g_h2d_next = 0, g_h2d_dev = -1;

int ncm_h2d_async(void *d, const void *h, size_t n) {
    int rc = ncm_ready();
    if (rc || n == 0) return rc;
    if (n > H2D_SLOT_BYTES || (g_h2d_pin && g_h2d_dev != ncm_device())) {
        mem_h2d(d, h, n);
        return ncm_ready();
    }
    if (!g_h2d_pin) {
        HIP_TRY(hipHostMalloc((void **)&g_h2d_pin, H2D_SLOTS * H2D_SLOT_BYTES, hipHostMallocDefault));
        for (int i = 0; i < H2D_SLOTS; i++) HIP_TRY(hipEventCreateWithFlags(&g_h2d_ev[i], hipEventDisableTiming));
        g_h2d_dev = ncm_device();
    }
    const int s = g_h2d_next;
    g_h2d_next = (s + 1) % H2D_SLOTS;
    if (g_h2d_used[s]) HIP_TRY(hipEventSynchronize(g_h2d_ev[s]));
    unsigned char *slot = g_h2d_pin + (size_t)s * H2D_SLOT_BYTES;
    memcpy(slot, h, n);
    HIP_TRY(hipMemcpyAsync(d, slot, n, hipMemcpyHostToDevice, g_stream));
    HIP_TRY(hipEventRecord(g_h2d_ev[s], g_stream));
    g_h2d_used[s] = 1;
    return 0;
}

void mem_d2d(void *d, const void *s, size_t n) {
    if (ncm_ready() || n == 0) return;
    hipError_t e = hipMemcpyAsync(d, s, n, hipMemcpyDeviceToDevice, g_stream);
    if (e == hipSuccess) e = hipStreamSynchronize(g_stream);
    if (e != hipSuccess) ncm_fail(NCM_E_HIP, "mem_d2d(%zu): %s", n, hipGetErrorString(e));
}

int ncm_copy_async(void *d, const void *s, size_t n) {
    if (n == 0) return 0;
    HIP_TRY(hipMemcpyAsync(d, s, n, hipMemcpyDeviceToDevice, g_stream));
    return 0;
}

int ncm_zero_async(void *d, size_t n) {
    if (n == 0) return 0;
    HIP_TRY(hipMemsetAsync(d, 0, n, g_stream));
    return 0;
}

void tensor_to_host(const Tensor *t, float *out) { mem_d2h(out, t->data, (size_t)t->n * sizeof(float)); }
void tensor_to_backend(Tensor *t, const float *in) { mem_h2d(t->data, in, (size_t)t->n * sizeof(float)); }

void *backend_to_host(const float *d, size_t nbytes) {
    void *h = malloc(nbytes ? nbytes : 1);
    if (!h) {
        ncm_fail(NCM_E_OOM, "backend_to_host(%zu)", nbytes);
        return NULL;
    }
    mem_d2h(h, d, nbytes);
    return h;
}

/* ---- bump arenas (tensor.c:268-365): 16-byte aligned, overflow is an error ---- */
typedef struct {
    unsigned char *base;
    size_t size, off;
} Arena;
static Arena g_arena, g_parena;

static float *arena_take(Arena *a, size_t n_floats, const char *what) {
    size_t need = n_floats * sizeof(float);
    size_t off = (a->off + 15) & ~(size_t)15;
    if (!a->base || off + need > a->size) {
        ncm_fail(NCM_E_OOM, "%s overflow (%zu > %zu MB)%s", what, (off + need) >> 20, a->size >> 20,
                 a->base ? "; raise NCM_ARENA_MB" : " (not initialised)");
        return NULL;
    }
    a->off = off + need;
    return (float *)(a->base + off);
}

void arena_free(void) {
    if (!g_arena.base) return;
    ncm_hip_free(g_arena.base);
    g_arena.base = NULL;
    g_arena.size = g_arena.off = 0;
}

void arena_init(size_t bytes) {
    arena_free();
    g_arena.base = (unsigned char *)ncm_hip_malloc(bytes);
    g_arena.size = g_arena.base ? bytes : 0;
    g_arena.off = 0;
}

void arena_init_default(void) {
    const char *e = getenv("NCM_ARENA_MB");
    size_t mb = e ? (size_t)atol(e) : 4096;
    if (mb < 64) mb = 64;
    arena_init(mb << 20);
}

float *arena_alloc(size_t n_floats) { return arena_take(&g_arena, n_floats, "arena"); }
void arena_reset(void) { g_arena.off = 0; }

void parena_init(size_t bytes) {
    if (g_parena.base) return;
    g_parena.base = (unsigned char *)ncm_hip_malloc(bytes);
    g_parena.size = g_parena.base ? bytes : 0;
    g_parena.off = 0;
}

float *parena_alloc(size_t n_floats) { return arena_take(&g_parena, n_floats, "parena"); }
