// vq.hip -- nearest-codeword search for cncm's multiscale residual quantiser
// (reference: rowwise_l2sq kernels.c:753-770 + host argmin vq.c:440-443 +
// residual update vq.c:476-498), bit-exact with the reference codes.
//
// The reference code of row i is the lowest j minimising
//     d2[i,j] = (float) sum_c ((double)x[i,c] - (double)E[j,c])^2
// (fp64, serial over c, no FMA; strict '<' scan).  The search runs in two
// stages:
//
// 1. vq_argmin_main -- an FP32-MFMA contraction s = x . E^T over all V
//    codewords with a fused running (best, index, second-best) per row of
//        e_j = |E_j|^2 - 2 x.E_j     (= d2 - |x|^2, same order as d2)
//    kept in registers; the R x V distance matrix is never written.  Every
//    e_j is within a proven bound eps_i of its exact value (worst-case fp32
//    dot-product error gamma_D |x||E_j| plus the roundings of |E_j|^2 and the
//    subtraction, doubled for safety).  When second - best exceeds
//    2 eps_i + one float ulp of the largest possible d2, every other codeword
//    is farther by more than an ulp in exact arithmetic, so the float d2 of
//    the winner is strictly smallest and the code is certain.
// 2. vq_rescore -- rows that fail the certificate (near-ties, exact ties,
//    non-finite inputs) are rescored with the reference arithmetic for all V
//    codewords, and the lowest index of the minimal float distance wins.
#include "ncm_dev.h"

#include <float.h>

struct VqArgs {
    const float *X;      // [rows, D] rows being quantised
    const float *E;      // [V, D] codebook
    const float *cn;     // [V]  (float) |E_j|^2, fp64 accumulated
    const float *xn;     // [rows] upper bound of |x_i|
    const unsigned *cmax_bits;  // upper bound of max_j |E_j| (float bits)
    int *idx;            // codes, written at idx[(row/L)*total + off + row%L]
    int *flag_list;      // rows needing the exact rescore
    int *flag_count;
    int rows, V, D;
    int L, total, off;
};

__device__ __forceinline__ int64_t code_slot(int row, int L, int total, int off) {
    return (int64_t)(row / L) * total + off + row % L;
}

// Merge of two (best, index, second) triples; ties on best keep the lower
// index and make the other best a second.
__device__ __forceinline__ void merge3(float &m1, int &i1, float &m2, float o1, int oi, float o2) {
    bool take = (o1 < m1) || (o1 == m1 && (unsigned)oi < (unsigned)i1);
    float lo = take ? m1 : o1;  // the best that loses
    if (take) { m1 = o1; i1 = oi; }
    m2 = fminf(fminf(m2, o2), lo);
}

// Minimum gap between best and second e that certifies the winner.
__device__ __forceinline__ float vq_threshold(float xn, float cm, int D) {
    const float u = 5.9604644775390625e-8f;  // 2^-24
    float du = (float)D * u;
    float gD = du / (1.0f - du);
    float eps = 2.0f * (2.0f * u * cm * cm + (2.0f * gD + 2.0f * u) * xn * cm + (float)D * 4.0f * FLT_MIN);
    float dmax = (xn + cm) * (xn + cm);
    float margin = 2.0f * u * dmax * 1.01f + 1e-12f * dmax + 1e-30f;
    return (2.0f * eps + margin) * 1.01f;
}

// counters[0] = flag count, counters[1] = bits of max |E_j|.
extern "C" __global__ void vq_init(unsigned *counters) {
    if (threadIdx.x == 0) { counters[0] = 0u; counters[1] = 0u; }
}

// cn[j] = (float) sum_c E[j,c]^2 (fp64); cmax = upper bound of max_j |E_j|.
extern "C" __global__ void __launch_bounds__(256)
vq_prep_codebook(const float *__restrict__ E, int V, int D, float *__restrict__ cn, unsigned *cmax_bits) {
    int j = blockIdx.x * 256 + threadIdx.x;
    float nrm = 0.f;
    if (j < V) {
        const float *e = E + (int64_t)j * D;
        double s = 0.0;
        for (int c = 0; c < D; ++c) s += (double)e[c] * (double)e[c];
        cn[j] = (float)s;
        nrm = (float)sqrt(s) * (1.0f + 1e-6f);
        if (!(nrm <= FLT_MAX)) nrm = __int_as_float(0x7f800000);  // NaN/inf -> +inf
    }
    // block max, then one atomic per block (non-negative floats order as uints)
    __shared__ float red[4];
    for (int o = 32; o > 0; o >>= 1) nrm = fmaxf(nrm, __shfl_xor(nrm, o, 64));
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = nrm;
    __syncthreads();
    if (threadIdx.x == 0) {
        float m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
        atomicMax(cmax_bits, __float_as_uint(m));
    }
}

// xn[i] = upper bound of |x_i| (one wave per row).
extern "C" __global__ void __launch_bounds__(256)
vq_rownorm(const float *__restrict__ X, int rows, int D, float *__restrict__ xn) {
    int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    int lane = threadIdx.x & 63;
    if (row >= rows) return;
    const float *x = X + (int64_t)row * D;
    double s = 0.0;
    for (int c = lane; c < D; c += 64) s += (double)x[c] * (double)x[c];
    s = wave_sum_d(s);
    if (lane == 0) {
        float v = (float)sqrt(s) * (1.0f + 1e-6f);
        if (!(v <= FLT_MAX)) v = __int_as_float(0x7f800000);
        xn[row] = v;
    }
}

// Stage 1.  Workgroup = 128 rows x all V codewords, 4 waves of 64x64 MFMA
// sub-tiles per 128-codeword tile, BK = 16; the (codeword tile, k slab)
// sequence is one double-buffered pipeline.
#define VQ_BM 128
#define VQ_BN 128
#define VQ_BK 16

template <bool VEC>
__device__ __forceinline__ void vq_main_body(const VqArgs &p) {
    constexpr int NT = 256, WM = 64, WN = 64, TM = 4, TN = 4;
    constexpr int LDA = VQ_BK + 4;
    constexpr int A_SZ = VQ_BM * LDA, B_SZ = VQ_BN * LDA;
    __shared__ __attribute__((aligned(16))) float smem[2 * (A_SZ + B_SZ)];
    __shared__ float red_m1[VQ_BM], red_m2[VQ_BM];
    __shared__ int red_i1[VQ_BM];

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int li = lane & 15, lg = lane >> 4;
    const int i0 = blockIdx.x * VQ_BM;

    const int nks = (p.D + VQ_BK - 1) / VQ_BK;
    const int nnt = (p.V + VQ_BN - 1) / VQ_BN;
    const int nsteps = nks * nnt;

    TileLoader<VQ_BM, VQ_BK, NT, VEC> la;
    TileLoader<VQ_BN, VQ_BK, NT, VEC> lb;

    float m1[TM * 4], m2[TM * 4];
    int i1[TM * 4];
#pragma unroll
    for (int s = 0; s < TM * 4; ++s) { m1[s] = INFINITY; m2[s] = INFINITY; i1[s] = -1; }

    f4 acc[TM][TN];
#pragma unroll
    for (int a = 0; a < TM; ++a)
#pragma unroll
        for (int b = 0; b < TN; ++b) acc[a][b] = f4{0.f, 0.f, 0.f, 0.f};

    auto gload = [&](int step) {
        int nt = step / nks, kt = step - nt * nks;
        la.load(p.X, p.D, i0, kt * VQ_BK, p.rows, p.D, tid);
        lb.load(p.E, p.D, nt * VQ_BN, kt * VQ_BK, p.V, p.D, tid);
    };

    gload(0);
    la.store(smem, tid);
    lb.store(smem + 2 * A_SZ, tid);
    __syncthreads();

    for (int st = 0; st < nsteps; ++st) {
        const int cur = st & 1;
        const bool more = st + 1 < nsteps;
        if (more) gload(st + 1);
        const float *a_s = smem + cur * A_SZ;
        const float *b_s = smem + 2 * A_SZ + cur * B_SZ;
        f4 ak[TM], bk[TN];
#pragma unroll
        for (int t = 0; t < TM; ++t) ak[t] = *(const f4 *)(a_s + (wm * WM + t * 16 + li) * LDA + 4 * lg);
#pragma unroll
        for (int t = 0; t < TN; ++t) bk[t] = *(const f4 *)(b_s + (wn * WN + t * 16 + li) * LDA + 4 * lg);
#pragma unroll
        for (int s = 0; s < 4; ++s)
#pragma unroll
            for (int a = 0; a < TM; ++a)
#pragma unroll
                for (int b = 0; b < TN; ++b) acc[a][b] = mfma4(ak[a][s], bk[b][s], acc[a][b]);

        const int nt = st / nks;
        if (st - nt * nks == nks - 1) {
            // codeword tile complete: fold e_j = cn_j - 2 s into the running triples
#pragma unroll
            for (int b = 0; b < TN; ++b) {
                const int j = nt * VQ_BN + wn * WN + b * 16 + li;
                if (j < p.V) {
                    const float cj = p.cn[j];
#pragma unroll
                    for (int a = 0; a < TM; ++a)
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            float e = cj - 2.0f * acc[a][b][r];
                            int s = a * 4 + r;
                            if (e < m1[s]) { m2[s] = m1[s]; m1[s] = e; i1[s] = j; }
                            else if (e < m2[s]) m2[s] = e;
                        }
                }
#pragma unroll
                for (int a = 0; a < TM; ++a) acc[a][b] = f4{0.f, 0.f, 0.f, 0.f};
            }
        }
        if (more) {
            la.store(smem + (cur ^ 1) * A_SZ, tid);
            lb.store(smem + 2 * A_SZ + (cur ^ 1) * B_SZ, tid);
        }
        __syncthreads();
    }

    // lanes sharing a row: the 16 li values of one lg group
#pragma unroll
    for (int s = 0; s < TM * 4; ++s) {
#pragma unroll
        for (int o = 1; o < 16; o <<= 1) {
            float o1 = __shfl_xor(m1[s], o, 64);
            float o2 = __shfl_xor(m2[s], o, 64);
            int oi = __shfl_xor(i1[s], o, 64);
            merge3(m1[s], i1[s], m2[s], o1, oi, o2);
        }
    }
    // the two waves (wn = 0, 1) sharing rows
    if (wn == 1 && li == 0) {
#pragma unroll
        for (int s = 0; s < TM * 4; ++s) {
            int lr = wm * WM + (s >> 2) * 16 + 4 * lg + (s & 3);
            red_m1[lr] = m1[s]; red_m2[lr] = m2[s]; red_i1[lr] = i1[s];
        }
    }
    __syncthreads();
    if (wn == 0 && li == 0) {
        const float cm = __uint_as_float(*p.cmax_bits);
#pragma unroll
        for (int s = 0; s < TM * 4; ++s) {
            int lr = wm * WM + (s >> 2) * 16 + 4 * lg + (s & 3);
            int row = i0 + lr;
            if (row >= p.rows) continue;
            merge3(m1[s], i1[s], m2[s], red_m1[lr], red_i1[lr], red_m2[lr]);
            float thr = vq_threshold(p.xn[row], cm, p.D);
            int64_t slot = code_slot(row, p.L, p.total, p.off);
            if (i1[s] >= 0 && m2[s] - m1[s] > thr) {
                p.idx[slot] = i1[s];
            } else {
                p.idx[slot] = -1;
                int f = atomicAdd(p.flag_count, 1);
                p.flag_list[f] = row;
            }
        }
    }
}

extern "C" __global__ void __launch_bounds__(256, 2) vq_argmin_main_v(VqArgs p) { vq_main_body<true>(p); }
extern "C" __global__ void __launch_bounds__(256, 2) vq_argmin_main_s(VqArgs p) { vq_main_body<false>(p); }

// The reference distance, bit for bit: fp64, serial over c, separate
// multiply and add roundings (kernels.c:760-765), then rounded to float.
__device__ __attribute__((noinline)) float exact_d2(const float *__restrict__ x, const float *__restrict__ e, int D) {
#pragma clang fp contract(off)
    double s = 0.0;
    for (int c = 0; c < D; ++c) {
        double d = (double)x[c] - (double)e[c];
        s = s + d * d;
    }
    return (float)s;
}

#define VQ_MAXD 4096

// Stage 2: one workgroup per flagged row, grid-stride over the flag list.
// Returns the reference's strict-'<' scan result: index 0 when d2[0] is NaN,
// otherwise the lowest index of the minimal non-NaN float distance.
extern "C" __global__ void __launch_bounds__(256)
vq_rescore(const float *__restrict__ X, const float *__restrict__ E, int V, int D,
           const int *__restrict__ flag_list, const unsigned *counters, int *idx,
           int L, int total, int off) {
    __shared__ float xs[VQ_MAXD];
    __shared__ float bv[4];
    __shared__ int bi[4];
    __shared__ int nan0;
    const int tid = threadIdx.x;
    const int n = (int)counters[0];
    for (int f = blockIdx.x; f < n; f += gridDim.x) {
        const int row = flag_list[f];
        const float *x = X + (int64_t)row * D;
        for (int c = tid; c < D; c += 256) xs[c] = x[c];
        __syncthreads();
        float best = INFINITY;
        int bidx = 0x7fffffff;
        for (int j = tid; j < V; j += 256) {
            float d = exact_d2(xs, E + (int64_t)j * D, D);
            if (j == 0) nan0 = d != d;
            if (d < best) { best = d; bidx = j; }
        }
        for (int o = 32; o > 0; o >>= 1) {
            float ov = __shfl_xor(best, o, 64);
            int oi = __shfl_xor(bidx, o, 64);
            if (ov < best || (ov == best && oi < bidx)) { best = ov; bidx = oi; }
        }
        if ((tid & 63) == 0) { bv[tid >> 6] = best; bi[tid >> 6] = bidx; }
        __syncthreads();
        if (tid == 0) {
            float b = bv[0];
            int i = bi[0];
            for (int w = 1; w < 4; ++w)
                if (bv[w] < b || (bv[w] == b && bi[w] < i)) { b = bv[w]; i = bi[w]; }
            if (nan0 || i == 0x7fffffff) i = 0;
            idx[code_slot(row, L, total, off)] = i;
        }
        __syncthreads();
    }
}

// d2[i,j] for the drop-in rowwise_l2sq: one thread per (i, j), reference
// arithmetic.  (The quantiser never materialises this matrix.)
extern "C" __global__ void __launch_bounds__(256)
l2sq_exact(const float *__restrict__ a, const float *__restrict__ b, float *__restrict__ d2,
           int64_t rows, int64_t cols, int C) {
    int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= rows * cols) return;
    int64_t r = i / cols, j = i % cols;
    d2[i] = exact_d2(a + r * C, b + j * C, C);
}

// Residual update of one level (vq.c:476-498 with identity resampling):
// q = E[code]; z_hat += q; z_rest -= q, in float.  On the first level z_hat
// starts from +0.0 as the reference's memset does, so z_hat = 0.0f + q.
extern "C" __global__ void __launch_bounds__(256)
vq_residual(const float *__restrict__ E, const int *__restrict__ idx, int rows, int V, int D,
            int L, int total, int off, int first, float *z_hat, float *z_rest) {
    int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (int64_t)rows * D) return;
    int row = (int)(i / D), c = (int)(i % D);
    int code = idx[code_slot(row, L, total, off)];
    if ((unsigned)code >= (unsigned)V) code = 0;  // never read outside E
    float q = E[(int64_t)code * D + c];
    float h = first ? 0.0f : z_hat[i];
    z_hat[i] = h + q;
    z_rest[i] = z_rest[i] - q;
}
