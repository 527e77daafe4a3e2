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
//    codewords with a fused running (best, index, second, index, third) per
//    row of
//        e_j = |E_j|^2 - 2 x.E_j     (= d2 - |x|^2, same order as d2)
//    kept in registers; the R x V distance matrix is never written.  Every
//    e_j is within a proven bound eps_i of its exact value (worst-case fp32
//    dot-product error gamma_D |x||E_j| plus the roundings of |E_j|^2 and the
//    subtraction, doubled for safety).  When second - best exceeds
//    2 eps_i + one float ulp of the largest possible d2, every other codeword
//    is farther by more than an ulp in exact arithmetic, so the float d2 of
//    the winner is strictly smallest and the code is certain.  When only
//    third - best exceeds it, the code is one of the two tracked codewords.
// 2. vq_rescore -- rows of the second kind get the two candidates' distances
//    in the reference arithmetic; the remaining rows (three or more
//    near-ties, exact ties, non-finite inputs) are rescored against all V
//    codewords, split over workgroups of 256 codewords whose (d2, index)
//    minima meet in a 64-bit atomicMin.  The lowest index of the minimal
//    float distance wins, as in the reference's strict '<' scan.
#include "ncm_dev.h"

#include <float.h>

struct VqArgs {
    const float *X;      // [rows, D] rows being quantised
    const float *E;      // [V, D] codebook
    const float *cn;     // [V]  (float) |E_j|^2, fp64 accumulated
    const float *xn;     // [rows] upper bound of |x_i|
    const unsigned *cmax_bits;  // upper bound of max_j |E_j| (float bits)
    int *idx;            // codes, written at idx[(row/L)*total + off + row%L]
    int *flag_list;      // rows needing the full exact rescore
    int *flag_count;
    int *pair_list;      // (row, i1, i2) of rows decided between two codewords
    int *pair_count;
    unsigned long long *keys;  // per full-rescore row: min (d2 bits, index)
    unsigned *done;            // per full-rescore row: finished codeword blocks
    int rows, V, D;
    int L, total, off;
};

__device__ __forceinline__ int64_t code_slot(int row, int L, int total, int off) {
    return (int64_t)(row / L) * total + off + row % L;
}

// Merge of two (best, index, second, index, third) lists: each side is
// sorted, and every value a side does not hold is >= its third.  Ties on a
// value keep the lower index first.
__device__ __forceinline__ void merge5(float &m1, int &i1, float &m2, int &i2, float &m3,
                                       float o1, int oi1, float o2, int oi2, float o3) {
    bool take = (o1 < m1) || (o1 == m1 && (unsigned)oi1 < (unsigned)i1);
    float a2 = take ? o2 : m2, a3 = take ? o3 : m3;  // rest of the winning side
    int ai2 = take ? oi2 : i2;
    float b1 = take ? m1 : o1, b2 = take ? m2 : o2;  // the losing side
    int bi1 = take ? i1 : oi1;
    if (take) { m1 = o1; i1 = oi1; }
    bool sec = (b1 < a2) || (b1 == a2 && (unsigned)bi1 < (unsigned)ai2);
    m3 = sec ? fminf(a2, b2) : fminf(a3, b1);
    m2 = sec ? b1 : a2;
    i2 = sec ? bi1 : ai2;
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

// counters[0] = full-rescore count, counters[1] = bits of max |E_j|,
// counters[2] = pair count.
extern "C" __global__ void vq_init(unsigned *counters) {
    if (threadIdx.x < 3) counters[threadIdx.x] = 0u;
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
    __shared__ float red_m1[VQ_BM], red_m2[VQ_BM], red_m3[VQ_BM];
    __shared__ int red_i1[VQ_BM], red_i2[VQ_BM];

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

    float m1[TM * 4], m2[TM * 4], m3[TM * 4];
    int i1[TM * 4], i2[TM * 4];
#pragma unroll
    for (int s = 0; s < TM * 4; ++s) {
        m1[s] = INFINITY; m2[s] = INFINITY; m3[s] = INFINITY; i1[s] = -1; i2[s] = -1;
    }

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
                            if (e < m1[s]) {
                                m3[s] = m2[s]; m2[s] = m1[s]; i2[s] = i1[s]; m1[s] = e; i1[s] = j;
                            } else if (e < m2[s]) {
                                m3[s] = m2[s]; m2[s] = e; i2[s] = j;
                            } else {
                                m3[s] = fminf(m3[s], e);
                            }
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
            float o3 = __shfl_xor(m3[s], o, 64);
            int oi1 = __shfl_xor(i1[s], o, 64);
            int oi2 = __shfl_xor(i2[s], o, 64);
            merge5(m1[s], i1[s], m2[s], i2[s], m3[s], o1, oi1, o2, oi2, o3);
        }
    }
    // the two waves (wn = 0, 1) sharing rows
    if (wn == 1 && li == 0) {
#pragma unroll
        for (int s = 0; s < TM * 4; ++s) {
            int lr = wm * WM + (s >> 2) * 16 + 4 * lg + (s & 3);
            red_m1[lr] = m1[s]; red_m2[lr] = m2[s]; red_m3[lr] = m3[s];
            red_i1[lr] = i1[s]; red_i2[lr] = i2[s];
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
            merge5(m1[s], i1[s], m2[s], i2[s], m3[s], red_m1[lr], red_i1[lr], red_m2[lr], red_i2[lr],
                   red_m3[lr]);
            float thr = vq_threshold(p.xn[row], cm, p.D);
            int64_t slot = code_slot(row, p.L, p.total, p.off);
            if (i1[s] >= 0 && m2[s] - m1[s] > thr) {
                p.idx[slot] = i1[s];
            } else if (i1[s] >= 0 && i2[s] >= 0 && m3[s] - m1[s] > thr) {
                p.idx[slot] = -1;
                int f = atomicAdd(p.pair_count, 1);
                p.pair_list[3 * f] = row;
                p.pair_list[3 * f + 1] = i1[s];
                p.pair_list[3 * f + 2] = i2[s];
            } else {
                p.idx[slot] = -1;
                int f = atomicAdd(p.flag_count, 1);
                p.flag_list[f] = row;
                p.keys[f] = ~0ull;
                p.done[f] = 0u;
            }
        }
    }
}

extern "C" __global__ void __launch_bounds__(256, 2) vq_argmin_main_v(VqArgs p) { vq_main_body<true>(p); }
extern "C" __global__ void __launch_bounds__(256, 2) vq_argmin_main_s(VqArgs p) { vq_main_body<false>(p); }

// The reference distance, bit for bit: fp64, serial over c, separate
// multiply and add roundings (kernels.c:760-765), then rounded to float.
// Operands are read 32 at a time so that a chunk's loads are in flight
// together ahead of the serial add chain.  VEC: D % 4 == 0 and both rows
// 16-byte aligned.
template <bool VEC>
__device__ __forceinline__ float exact_d2(const float *__restrict__ x, const float *__restrict__ e, int D) {
#pragma clang fp contract(off)
    constexpr int CH = 32;
    double s = 0.0;
    int c = 0;
    for (; c + CH <= D; c += CH) {
        float xv[CH], ev[CH];
        if (VEC) {
#pragma unroll
            for (int q = 0; q < CH / 4; ++q) {
                f4 a = *(const f4 *)(x + c + 4 * q), b = *(const f4 *)(e + c + 4 * q);
#pragma unroll
                for (int t = 0; t < 4; ++t) { xv[4 * q + t] = a[t]; ev[4 * q + t] = b[t]; }
            }
        } else {
#pragma unroll
            for (int t = 0; t < CH; ++t) { xv[t] = x[c + t]; ev[t] = e[c + t]; }
        }
#pragma unroll
        for (int t = 0; t < CH; ++t) {
            double d = (double)xv[t] - (double)ev[t];
            s = s + d * d;
        }
    }
    for (; c < D; ++c) {
        double d = (double)x[c] - (double)e[c];
        s = s + d * d;
    }
    return (float)s;
}

#define VQ_MAXD 4096
#define RS_PAIRS 128  // pair rows per rescore unit, two lanes per row

// Stage 2, grid-stride over units: first the pair rows, RS_PAIRS per unit
// (lane 2k and 2k+1 score the two candidates of row k), then one unit per
// (full-rescore row, block of 256 codewords).  A full row's blocks fold
// (float bits of d2) << 32 | j into keys[f] with atomicMin -- d2 >= 0, so
// the bits order as the floats -- and the last block to finish writes the
// code.  NaN distances never win; a NaN at index 0 is key 0, because the
// reference scan then never leaves index 0.
extern "C" __global__ void __launch_bounds__(256)
vq_rescore(const float *__restrict__ X, const float *__restrict__ E, int V, int D, int vec,
           const int *__restrict__ flag_list, const int *__restrict__ pair_list,
           const unsigned *counters, unsigned long long *keys, unsigned *done, int *idx, int L,
           int total, int off) {
    __shared__ __attribute__((aligned(16))) float xs[VQ_MAXD];
    const int tid = threadIdx.x;
    const int n_full = (int)counters[0], n_pair = (int)counters[2];
    const int nb = (V + 255) / 256;
    const int64_t pu = (n_pair + RS_PAIRS - 1) / RS_PAIRS;
    const int64_t units = pu + (int64_t)n_full * nb;
    for (int64_t u = blockIdx.x; u < units; u += gridDim.x) {
        if (u < pu) {
            const int k = (int)u * RS_PAIRS + (tid >> 1);
            const bool ok = k < n_pair;
            float d = INFINITY;
            int j = 0x7fffffff, row = 0;
            if (ok) {
                row = pair_list[3 * k];
                j = pair_list[3 * k + 1 + (tid & 1)];
                const float *x = X + (int64_t)row * D, *e = E + (int64_t)j * D;
                d = vec ? exact_d2<true>(x, e, D) : exact_d2<false>(x, e, D);
            }
            float od = __shfl_xor(d, 1, 64);
            int oj = __shfl_xor(j, 1, 64);
            if (od < d || (od == d && oj < j)) { d = od; j = oj; }
            if (ok && (tid & 1) == 0) idx[code_slot(row, L, total, off)] = j;
        } else {
            const int64_t w = u - pu;
            const int f = (int)(w / nb), b = (int)(w - (int64_t)f * nb);
            const int row = flag_list[f];
            const float *x = X + (int64_t)row * D;
            for (int c = tid; c < D; c += 256) xs[c] = x[c];
            __syncthreads();
            const int j = b * 256 + tid;
            unsigned long long key = ~0ull;
            if (j < V) {
                const float *e = E + (int64_t)j * D;
                float d = vec ? exact_d2<true>(xs, e, D) : exact_d2<false>(xs, e, D);
                if (d == d) key = ((unsigned long long)__float_as_uint(d) << 32) | (unsigned)j;
                else if (j == 0) key = 0ull;
            }
            for (int o = 32; o > 0; o >>= 1) {
                unsigned long long ok = __shfl_xor(key, o, 64);
                key = ok < key ? ok : key;
            }
            if ((tid & 63) == 0 && key != ~0ull) atomicMin(&keys[f], key);
            __threadfence();
            __syncthreads();
            if (tid == 0 && atomicAdd(&done[f], 1u) == (unsigned)(nb - 1)) {
                __threadfence();
                unsigned long long k = atomicMin(&keys[f], ~0ull);  // the final value
                idx[code_slot(row, L, total, off)] = k == ~0ull ? 0 : (int)(unsigned)k;
            }
            __syncthreads();
        }
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
    d2[i] = exact_d2<false>(a + r * C, b + j * C, C);
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
