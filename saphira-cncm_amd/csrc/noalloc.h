/* noalloc.h -- the fixed device array behind the allocation-free VQ search
 * (noalloc_scratch.cpp) and the limits it sets. */
#ifndef NCM_NOALLOC_H
#define NCM_NOALLOC_H

/* vq_argmin_noalloc limits: rows <= 2^18 and V <= 2^16 fit the VQ search's
 * per-call scratch (counters | |E_j|^2 [V] | |x_i| [rows] | flagged rows |
 * row pairs | rescore keys | rescore counters, each 256-byte aligned) in
 * 9 MiB: 256 + 4 V + 32 rows + 5 * 255 bytes at most. */
#define NCM_NOALLOC_MAX_ROWS (1 << 18)
#define NCM_NOALLOC_MAX_V (1 << 16)
#define NCM_NOALLOC_SCRATCH_BYTES (9u << 20)

#ifdef __cplusplus
extern "C" {
#endif
/* Looks up this device's address of the array (device current); 0 or a
 * hipError_t code. */
int ncm_noalloc_setup(int device);
/* The address found by ncm_noalloc_setup for `device`, or NULL with *err
 * set to the lookup's error (0 when setup never ran). */
void *ncm_noalloc_scratch(int device, int *err);
const char *ncm_noalloc_error_string(int err);
#ifdef __cplusplus
}
#endif

#endif
