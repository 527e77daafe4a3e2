// ops.hip -- row-wise and elementwise kernels around the GEMMs.
#include "ncm_dev.h"

// Greedy id: per row the reference's strict '>' scan from index 0
// (kernels.c:731-735): index 0 when x[0] is NaN, otherwise the lowest index
// of the maximal non-NaN value (0 when no value exceeds x[0] = -inf).
extern "C" __global__ void __launch_bounds__(256)
argmax_rows_k(const float *__restrict__ x, int n, int *__restrict__ idx) {
    __shared__ float bv[4];
    __shared__ int bi[4];
    const int tid = threadIdx.x;
    const float *xr = x + (int64_t)blockIdx.x * n;
    float best = -INFINITY;
    int bidx = 0x7fffffff;
    for (int j = tid; j < n; j += 256) {
        float v = xr[j];
        if (v > best) { best = v; bidx = j; }
    }
    for (int o = 32; o > 0; o >>= 1) {
        float ov = __shfl_xor(best, o, 64);
        int oi = __shfl_xor(bidx, o, 64);
        if (ov > best || (ov == best && oi < bidx)) { best = ov; bidx = oi; }
    }
    if ((tid & 63) == 0) { bv[tid >> 6] = best; bi[tid >> 6] = bidx; }
    __syncthreads();
    if (tid == 0) {
        float b = bv[0];
        int i = bi[0];
        for (int w = 1; w < 4; ++w)
            if (bv[w] > b || (bv[w] == b && bi[w] < i)) { b = bv[w]; i = bi[w]; }
        float x0 = xr[0];
        if (x0 != x0 || i == 0x7fffffff) i = 0;
        idx[blockIdx.x] = i;
    }
}
