// vq.hip -- nearest-codeword search for cncm's multiscale residual quantiser
// (reference: rowwise_l2sq kernels.c:753-770 + host argmin vq.c:440-443 +
// residual update vq.c:476-498), bit-exact with the reference codes.
//
// The reference code of row i is the lowest j minimising
//     d2[i,j] = (float) sum_c ((double)x[i,c] - (double)E[j,c])^2
// (fp64, serial over c, no FMA; strict '<' scan).  The search runs in two
// stages:
//
// 1. vq_argmin_main_* -- an FP32-MFMA contraction s = x . E^T over all V
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
#include "mfma_slab.h"

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
// One wave per codeword at a time (lanes over c, float4 loads when vec), so
// the rows are read coalesced and the fp64 sums run 64 wide; cn differs from
// a serial sum only in the fp64 rounding order, far inside the screen's bound
// for the rounding of |E_j|^2.  Waves stride over the codebook so that at
// most gridDim.x (<= 256) atomics meet on cmax: one per codeword group of 4
// had serialised there.
extern "C" __global__ void __launch_bounds__(256)
vq_prep_codebook_w(const float *__restrict__ E, int V, int D, int vec, float *__restrict__ cn,
                   unsigned *cmax_bits) {
    const int lane = threadIdx.x & 63;
    float nrm = 0.f;
    for (int j = blockIdx.x * 4 + (threadIdx.x >> 6); j < V; j += gridDim.x * 4) {
        const float *e = E + (int64_t)j * D;
        double s = 0.0;
        if (vec) {
            for (int c = 4 * lane; c < D; c += 256) {
                const f4 v = *(const f4 *)(e + c);
                s += ((double)v.x * (double)v.x + (double)v.y * (double)v.y) +
                     ((double)v.z * (double)v.z + (double)v.w * (double)v.w);
            }
        } else {
            for (int c = lane; c < D; c += 64) s += (double)e[c] * (double)e[c];
        }
        s = wave_sum_d(s);
        if (lane == 0) cn[j] = (float)s;
        float n = (float)sqrt(s) * (1.0f + 1e-6f);
        if (!(n <= FLT_MAX)) n = __int_as_float(0x7f800000);  // NaN/inf -> +inf
        nrm = fmaxf(nrm, n);
    }
    __shared__ float red[4];
    if (lane == 0) red[threadIdx.x >> 6] = nrm;
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
    if ((D & 3) == 0 && ((uintptr_t)X & 15) == 0) {   // float4 loads
        for (int c = 4 * lane; c < D; c += 256) {
            const f4 v = *(const f4 *)(x + c);
            s += ((double)v.x * (double)v.x + (double)v.y * (double)v.y) +
                 ((double)v.z * (double)v.z + (double)v.w * (double)v.w);
        }
    } else {
        for (int c = lane; c < D; c += 64) s += (double)x[c] * (double)x[c];
    }
    s = wave_sum_d(s);
    if (lane == 0) {
        float v = (float)sqrt(s) * (1.0f + 1e-6f);
        if (!(v <= FLT_MAX)) v = __int_as_float(0x7f800000);
        xn[row] = v;
    }
}

// Running (best, index, second, index, third) of one row slot; j arrives in
// increasing order, so the strict '<' keeps the lowest index among equal e.
#define VQ_TRACK(s, e, j)                                                         \
    do {                                                                          \
        if ((e) < m1[s]) {                                                        \
            m3[s] = m2[s]; m2[s] = m1[s]; i2[s] = i1[s]; m1[s] = (e); i1[s] = (j); \
        } else if ((e) < m2[s]) {                                                 \
            m3[s] = m2[s]; m2[s] = (e); i2[s] = (j);                              \
        } else {                                                                  \
            m3[s] = fminf(m3[s], (e));                                            \
        }                                                                         \
    } while (0)

// Folds the per-lane lists of NS row slots (rows lrow(s) of the workgroup's
// tile) over the 16 lanes li that share a row and the two waves wn = 0, 1,
// then decides each row: certified code, pair rescore or full rescore.
template <int NS, typename RowOf>
__device__ __forceinline__ void vq_decide(const VqArgs &p, float (&m1)[NS], int (&i1)[NS], float (&m2)[NS],
                                          int (&i2)[NS], float (&m3)[NS], int i0, int wn, int li,
                                          float *red_m1, float *red_m2, float *red_m3, int *red_i1,
                                          int *red_i2, RowOf lrow) {
#pragma unroll
    for (int s = 0; s < NS; ++s) {
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
    if (wn == 1 && li == 0) {
#pragma unroll
        for (int s = 0; s < NS; ++s) {
            const int lr = lrow(s);
            red_m1[lr] = m1[s]; red_m2[lr] = m2[s]; red_m3[lr] = m3[s];
            red_i1[lr] = i1[s]; red_i2[lr] = i2[s];
        }
    }
    __syncthreads();
    if (wn == 0 && li == 0) {
        const float cm = __uint_as_float(*p.cmax_bits);
#pragma unroll
        for (int s = 0; s < NS; ++s) {
            const int lr = lrow(s);
            const int row = i0 + lr;
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

// Register-staged slab loads for the scalar screen: the same [64 rows][32 k]
// swizzled slab as the direct-to-LDS loads (mfma_slab.h), any D and
// alignment.  Thread t stages float4 groups q = t and t + 256 (row q / 8,
// group q % 8); elements outside the rows or past D read zero.
struct VqStage {
    f4 v[2];
    __device__ __forceinline__ void load(const float *__restrict__ src, int ld, int row0, int nrows, int k0, int tid) {
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            const int q = tid + 256 * e, r = q >> 3, k = k0 + 4 * (q & 7);
            f4 x = {0.f, 0.f, 0.f, 0.f};
            if (row0 + r < nrows) {
                const float *sp = src + (int64_t)(row0 + r) * ld + k;
#pragma unroll
                for (int c = 0; c < 4; ++c)
                    if (k + c < ld) x[c] = sp[c];
            }
            v[e] = x;
        }
    }
    __device__ __forceinline__ void store(float *slab, int tid) const {
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            const int q = tid + 256 * e, r = q >> 3, g = q & 7;
            *(f4 *)(slab + r * GEMM_BK + 4 * (g ^ (r & 7))) = v[e];
        }
    }
};

// Stage 1: a workgroup owns 64 rows and sweeps all V codewords in tiles of
// 64; the (codeword tile, k slab) pairs form one stream of [64][32] slabs in
// two LDS stages.  Each wave owns 32 rows x 32 codewords of a tile (2 x 2
// MFMA blocks, fragments as in the linear GEMM); after a tile's last slab the
// accumulators are folded into the running lists.  Four workgroups share a CU.
//   DMA (vectorised: D % 4 == 0, 16-byte aligned rows): the linear GEMM's
//     direct-to-LDS pipeline -- one barrier per slab, fragment reads one
//     chunk ahead of the MFMAs, the loads of the slab after next issued after
//     the barrier.  Buffer descriptors are rebased on the workgroup's rows and
//     on each codeword tile, sized to the rows that exist, so rows past either
//     end read zero (and are never folded or written).
//   register-staged (any D, any alignment): the next slab's loads are issued
//     before this slab's MFMAs and stored to the other stage after them.
template <bool DMA>
__device__ __forceinline__ void vq_screen_body(const VqArgs &p) {
    __shared__ __attribute__((aligned(16))) float sm[4 * D_SLAB];  // [stage][X | E]
    __shared__ float red_m1[64], red_m2[64], red_m3[64];
    __shared__ int red_i1[64], red_i2[64];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1, li = lane & 15, lg = lane >> 4;
    const int i0 = blockIdx.x * 64;
    const int ld = p.D;
    const int nks = (p.D + GEMM_BK - 1) / GEMM_BK;
    const int ntiles = (p.V + 63) / 64;
    const int nsteps = nks * ntiles;
    const __attribute__((address_space(1))) float *cn = (const __attribute__((address_space(1))) float *)p.cn;

    float m1[8], m2[8], m3[8];
    int i1[8], i2[8];
#pragma unroll
    for (int s = 0; s < 8; ++s) {
        m1[s] = INFINITY; m2[s] = INFINITY; m3[s] = INFINITY; i1[s] = -1; i2[s] = -1;
    }
    f4 acc[2][2];
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int b = 0; b < 2; ++b) acc[a][b] = f4{0.f, 0.f, 0.f, 0.f};
    auto mfmas = [&](const float (&fa)[2][4], const float (&fb)[2][4]) {
#pragma unroll
        for (int s = 0; s < 4; ++s)
#pragma unroll
            for (int a = 0; a < 2; ++a)
#pragma unroll
                for (int b = 0; b < 2; ++b) acc[a][b] = mfma4(fa[a][s], fb[b][s], acc[a][b]);
    };
    // |E_j|^2 of the lane's two codeword columns, one tile ahead
    float cj[2];
    auto load_cn = [&](int nt) {
#pragma unroll
        for (int b = 0; b < 2; ++b) {
            const int j = nt * 64 + wn * 32 + b * 16 + li;
            cj[b] = j < p.V ? cn[j] : 0.f;
        }
    };
    int nt = 0, kt = 0;
    // after each slab: a finished codeword tile folds e_j = |E_j|^2 - 2 x.E_j
    auto advance = [&]() {
        if (++kt < nks) return;
        kt = 0;
        const float c[2] = {cj[0], cj[1]};
        load_cn(nt + 1);
#pragma unroll
        for (int b = 0; b < 2; ++b) {
            const int j = nt * 64 + wn * 32 + b * 16 + li;
            if (j < p.V) {
#pragma unroll
                for (int a = 0; a < 2; ++a)
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const float e = c[b] - 2.0f * acc[a][b][r];
                        VQ_TRACK(a * 4 + r, e, j);
                    }
            }
#pragma unroll
            for (int a = 0; a < 2; ++a) acc[a][b] = f4{0.f, 0.f, 0.f, 0.f};
        }
        ++nt;
    };

    float *const s0 = sm, *const s1 = sm + 2 * D_SLAB;
    float f0a[2][4], f0b[2][4], f1a[2][4], f1b[2][4];
    load_cn(0);
    if constexpr (DMA) {
        const __amdgpu_buffer_rsrc_t ra =
            make_rsrc(p.X + (int64_t)i0 * ld, (unsigned)(min(p.rows - i0, 64) * ld * 4));
        DSlab<true> la, lb;
        la.init(wave, lane, ld, 0, 64, p.D);
        lb.init(wave, lane, ld, 0, 64, p.D);
        // the load stream runs two slabs ahead of the compute stream
        int lnt = 0, lkt = 0;
        auto issue = [&](float *stage) {
            const int nr = min(max(p.V - lnt * 64, 0), 64);
            const __amdgpu_buffer_rsrc_t rb =
                make_rsrc(nr ? p.E + (int64_t)lnt * 64 * ld : p.E, (unsigned)(nr * ld * 4));
            la.load(ra, stage, wave, lkt * GEMM_BK, ld);
            lb.load(rb, stage + D_SLAB, wave, lkt * GEMM_BK, ld);
            if (++lkt == nks) { lkt = 0; ++lnt; }
        };
        issue(s0);
        __builtin_amdgcn_s_waitcnt(0x0f70);   // vmcnt(0)
        __syncthreads();
        d_frags<true>(s0, wm, li, lg, 0, f0a);
        d_frags<true>(s0 + D_SLAB, wn, li, lg, 0, f0b);
        issue(s1);
        auto step = [&](float *cs, float *ns) {
            d_frags<true>(cs, wm, li, lg, 1, f1a);
            d_frags<true>(cs + D_SLAB, wn, li, lg, 1, f1b);
            __builtin_amdgcn_sched_barrier(0);
            mfmas(f0a, f0b);
            __builtin_amdgcn_sched_barrier(0);
            __builtin_amdgcn_s_waitcnt(0x0f70);   // vmcnt(0): this wave's loads of the next slab
            __syncthreads();
            d_frags<true>(ns, wm, li, lg, 0, f0a);
            d_frags<true>(ns + D_SLAB, wn, li, lg, 0, f0b);
            __builtin_amdgcn_sched_barrier(0);
            issue(cs);
            __builtin_amdgcn_sched_barrier(0);
            mfmas(f1a, f1b);
            __builtin_amdgcn_sched_barrier(0);
            advance();
        };
        for (int st = 0; st < nsteps; st += 2) {
            step(s0, s1);
            if (st + 1 < nsteps) step(s1, s0);
        }
        // No load may still be writing LDS when the workgroup ends.
        __builtin_amdgcn_s_waitcnt(0x0f70);
    } else {
        VqStage ga, gb;
        int lnt = 0, lkt = 0;
        auto fetch = [&]() {
            ga.load(p.X, ld, i0, p.rows, lkt * GEMM_BK, tid);
            gb.load(p.E, ld, lnt * 64, p.V, lkt * GEMM_BK, tid);
            if (++lkt == nks) { lkt = 0; ++lnt; }
        };
        fetch();
        ga.store(s0, tid);
        gb.store(s0 + D_SLAB, tid);
        __syncthreads();
        for (int st = 0; st < nsteps; ++st) {
            float *const cs = (st & 1) ? s1 : s0, *const ns = (st & 1) ? s0 : s1;
            const bool more = st + 1 < nsteps;
            if (more) fetch();
            d_frags<true>(cs, wm, li, lg, 0, f0a);
            d_frags<true>(cs + D_SLAB, wn, li, lg, 0, f0b);
            d_frags<true>(cs, wm, li, lg, 1, f1a);
            d_frags<true>(cs + D_SLAB, wn, li, lg, 1, f1b);
            mfmas(f0a, f0b);
            mfmas(f1a, f1b);
            advance();
            if (more) {
                ga.store(ns, tid);
                gb.store(ns + D_SLAB, tid);
            }
            __syncthreads();
        }
    }
    vq_decide<8>(p, m1, i1, m2, i2, m3, i0, wn, li, red_m1, red_m2, red_m3, red_i1, red_i2,
                 [&](int s) { return wm * 32 + (s >> 2) * 16 + 4 * lg + (s & 3); });
}

extern "C" __global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4)))
vq_argmin_main_v(VqArgs p) { vq_screen_body<true>(p); }
extern "C" __global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4)))
vq_argmin_main_s(VqArgs p) { vq_screen_body<false>(p); }

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

// Soft assignment (vq.c:400-431), step 1, one thread per row of the distance
// matrix dd [rows][V]: m = mean of the row (fp64, index order, as the
// reference's serial loop); m > 0 gives T = tau * m, bv = the row minimum and
// acc = sum_j exp(-(d_j - bv) / T) (index order) in st[3r..3r+2] and flag 1;
// otherwise flag 0 (argmin, no draw).
extern "C" __global__ void __launch_bounds__(256)
vq_soft_stats(const float *__restrict__ dd, int rows, int V, double tau, double *__restrict__ st,
              unsigned char *__restrict__ flag) {
#pragma clang fp contract(off)
    const int r = blockIdx.x * 256 + threadIdx.x;
    if (r >= rows) return;
    const float *d = dd + (int64_t)r * V;
    double m = 0;
    for (int j = 0; j < V; j++) m += (double)d[j];
    m /= V;
    if (!(m > 0)) {
        flag[r] = 0;
        return;
    }
    const double T = tau * m;
    double bv = d[0];
    for (int j = 1; j < V; j++)
        if ((double)d[j] < bv) bv = d[j];
    double acc = 0;
    for (int j = 0; j < V; j++) acc += exp(-((double)d[j] - bv) / T);
    st[3 * r] = T;
    st[3 * r + 1] = bv;
    st[3 * r + 2] = acc;
    flag[r] = 1;
}

// Step 2: u[r] >= 0 is the row's uniform draw (rng >> 11) * 2^-53: the code
// is the first j whose running sum of exp(-(d_j - bv) / T) exceeds u * acc
// (V - 1 if none); u[r] < 0 takes the argmin (first minimum).  The code goes to
// idx[(r / tl) * total + off + r % tl].  The host's exp (glibc, which the
// reference calls) and the device's may differ by an ulp or two per term, so
// the sums the draw is compared with are known to within
// eta = (V + 4) 2^-50 acc (two ulps per term plus one rounding per addition,
// doubled); near[r] = 1 marks a draw within eta of the running sum it was
// decided on (the chosen code's or the one before), which the host then
// decides again with its own exp.
extern "C" __global__ void __launch_bounds__(256)
vq_soft_pick(const float *__restrict__ dd, int rows, int V, const double *__restrict__ st,
             const double *__restrict__ u, int *__restrict__ idx, int tl, int total, int off,
             unsigned char *__restrict__ near) {
#pragma clang fp contract(off)
    const int r = blockIdx.x * 256 + threadIdx.x;
    if (r >= rows) return;
    const float *d = dd + (int64_t)r * V;
    const double ur = u[r];
    int bi = 0;
    unsigned char nr = 0;
    if (ur < 0) {
        float bv = d[0];
        for (int j = 1; j < V; j++)
            if (d[j] < bv) {
                bv = d[j];
                bi = j;
            }
    } else {
        const double T = st[3 * r], bv = st[3 * r + 1], acc = st[3 * r + 2], draw = ur * acc;
        const double eta = (double)(V + 4) * 0x1p-50 * acc;
        double csum = 0, prev = 0;
        bi = V - 1;
        for (int j = 0; j < V; j++) {
            prev = csum;
            csum += exp(-((double)d[j] - bv) / T);
            if (draw < csum) {
                bi = j;
                break;
            }
        }
        nr = fabs(draw - csum) <= eta || (bi > 0 && fabs(draw - prev) <= eta);
    }
    idx[(int64_t)(r / tl) * total + off + r % tl] = bi;
    near[r] = nr;
}

// EMA codebook step (vq.c:717-745), one thread per (code v, column d): the
// fp64 sum of the level's input rows holding code v (rows listed in row order,
// list[start[v] .. start[v + 1])), w = (float)(decay w + (1 - decay) sum), and
// the codebook E = (float)(w / sm[v]).
extern "C" __global__ void __launch_bounds__(256)
vq_ema_codebook(const float *__restrict__ x, const int *__restrict__ start, const int *__restrict__ list,
                const double *__restrict__ sm, float *__restrict__ w, float *__restrict__ E, int V, int D,
                double decay) {
#pragma clang fp contract(off)
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (int64_t)V * D) return;
    const int v = (int)(i / D), d = (int)(i - (int64_t)v * D);
    double sum = 0;
    for (int k = start[v]; k < start[v + 1]; k++) sum += (double)x[(int64_t)list[k] * D + d];
    const double keep = decay * (double)w[i], add = (1 - decay) * sum;
    const float nw = (float)(keep + add);
    w[i] = nw;
    E[i] = (float)((double)nw / sm[v]);
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

// The same on float4 groups (D % 4 == 0, 16-byte aligned E, z_hat, z_rest):
// the same float operations per element, the row and code found once per
// float4 in 32-bit arithmetic (the per-element kernel's 64-bit division and
// modulo were most of its time).
extern "C" __global__ void __launch_bounds__(256)
vq_residual4(const float *__restrict__ E, const int *__restrict__ idx, int rows, int V, int D, int L, int total,
             int off, int first, float *z_hat, float *z_rest) {
#pragma clang fp contract(off)
    const int per = D >> 2;
    const unsigned i4 = blockIdx.x * 256u + threadIdx.x;
    if (i4 >= (unsigned)rows * (unsigned)per) return;
    const int row = (int)(i4 / (unsigned)per), c = (int)(i4 - (unsigned)row * per) * 4;
    int code = idx[code_slot(row, L, total, off)];
    if ((unsigned)code >= (unsigned)V) code = 0;  // never read outside E
    const f4 q = *(const f4 *)(E + (int64_t)code * D + c);
    f4 *zh = (f4 *)(z_hat + (int64_t)row * D + c), *zr = (f4 *)(z_rest + (int64_t)row * D + c);
    const f4 h = first ? f4{0.f, 0.f, 0.f, 0.f} : *zh, r = *zr;
    *zh = h + q;
    *zr = r - q;
}

// ---------------------------------------------------------------- the full quantizer
// Resampling, convolutions and blends of src/vq.c's general multiscale path
// (per-level lengths, Phi, the learned level-0 cascade, refine convs), on
// [B][T][D] tensors (the reference's BLD layout) with the reference's
// arithmetic: fp64 accumulators in its loop orders, separate multiply and
// add roundings (no contraction), float results.  Bit-exact with the CPU.

// kernels.c:681-700 area interpolation, one thread per output (b, t, d);
// output row t of sequence b goes to y row b * ystride + yoff + t
extern "C" __global__ void __launch_bounds__(256)
vqf_area(const float *__restrict__ x, float *__restrict__ y, int B, int Tin, int Tout, int D, int ystride, int yoff) {
#pragma clang fp contract(off)
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (int64_t)B * Tout * D) return;
    const int d = (int)(i % D), t = (int)((i / D) % Tout), b = (int)(i / ((int64_t)D * Tout));
    int64_t s = (int64_t)((double)t * Tin / Tout);
    int64_t e = (int64_t)ceil((double)(t + 1) * Tin / Tout);
    if (e <= s) e = s + 1;
    if (s < 0) s = 0;
    if (e > Tin) e = Tin;
    double acc = 0.0;
    for (int64_t k = s; k < e; ++k) acc += (double)x[((int64_t)b * Tin + k) * D + d];
    y[((int64_t)b * ystride + yoff + t) * D + d] = (float)(acc / (double)(e - s));
}

// kernels.c:702-727 linear interpolation (align_corners = False; a length-1
// side averages), one thread per output
extern "C" __global__ void __launch_bounds__(256)
vqf_linear(const float *__restrict__ x, float *__restrict__ y, int B, int Tin, int Tout, int D) {
#pragma clang fp contract(off)
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (int64_t)B * Tout * D) return;
    const int d = (int)(i % D), t = (int)((i / D) % Tout), b = (int)(i / ((int64_t)D * Tout));
    const float *xc = x + (int64_t)b * Tin * D + d;
    if (Tout == 1 || Tin == 1) {
        double acc = 0.0;
        for (int k = 0; k < Tin; ++k) acc += (double)xc[(int64_t)k * D];
        y[i] = (float)(acc / Tin);
        return;
    }
    const double scale = (double)Tin / Tout;
    const double src = (t + 0.5) * scale - 0.5;
    const int64_t s0 = (int64_t)floor(src), s1 = s0 + 1;
    const double w1 = src - (double)s0, w0 = 1.0 - w1;
    const double v0 = xc[(s0 < 0 ? 0 : (s0 >= Tin ? Tin - 1 : s0)) * (int64_t)D];
    const double v1 = xc[(s1 < 0 ? 0 : (s1 >= Tin ? Tin - 1 : s1)) * (int64_t)D];
    y[i] = (float)(w0 * v0 + w1 * v1);
}

// conv1d (kernels.c:546-566; W [Cout][Cin][K]) or, with TR, ConvTranspose1d
// (kernels.c:568-590; W [Cin][Cout][K]) over x [B][T][Cin] into y [B][To][Cout]:
//   y = (float)(bias + sum over ci (outer), k (inner) of (double) x * W)
// A workgroup computes 64 output channels x 16 positions of one b; thread
// (co, g) carries the 4 positions 16 t0 + 4 g + j as 4 independent fp64
// chains, each in the reference's order.  Per chunk of input channels the
// weights are staged in LDS as [ci][k][co] (lanes read consecutive co) and
// the input window of the 16 positions as doubles [pos][ci] (a wave's lanes
// read one address).
//
// conv1d skips no term inside the loop: the window covers every position
// the taps touch, with +0.0 outside [0, T), so a tap the reference skips
// adds a signed zero.  Adding +-0 leaves a non-zero chain unchanged, and a
// zero chain can only change sign, which every later non-zero term undoes;
// so a result can differ from the reference's only when the final chain is
// exactly zero -- those few outputs are recomputed with the reference's
// skips (vqf_conv_exact).
#define VQF_KMAX 16
#define VQF_WP 65      // LDS row pitch of the staged weights (odd: conflict-free transposing stores)
#define VQF_WS (128 * VQF_WP)
#define VQF_XS 2048

__device__ double vqf_conv_exact(const float *__restrict__ xb, const float *__restrict__ W, const float *__restrict__ bias,
                                 int T, int Cin, int co, int K, int stride, int pad, int t) {
#pragma clang fp contract(off)
    double acc = bias ? (double)bias[co] : 0.0;
    for (int ci = 0; ci < Cin; ++ci)
        for (int k = 0; k < K; ++k) {
            const int ti = t * stride + k - pad;
            if (ti < 0 || ti >= T) continue;
            acc += (double)xb[(int64_t)ti * Cin + ci] * (double)W[((int64_t)co * Cin + ci) * K + k];
        }
    return acc;
}

template <bool TR, int KC, bool S1K3>
__device__ __forceinline__ void vqf_conv_body(const float *__restrict__ x, const float *__restrict__ W,
                                              const float *__restrict__ bias, float *__restrict__ y, int T,
                                              int Cin, int Cout, int Krt, int stride, int pad, int To) {
#pragma clang fp contract(off)
    __shared__ float ws[VQF_WS];
    __shared__ double xs[VQF_XS];
    const int K = KC > 0 ? KC : Krt;
    const int tid = threadIdx.x, col = tid & 63, g = tid >> 6;
    const int co0 = blockIdx.x * 64, t0 = blockIdx.y * 16, b = blockIdx.z;
    const int co = co0 + col;
    // input positions the 16 outputs read: [plo, phi] (conv1d: unclamped, padded with zeros)
    int plo, phi;
    if (TR) {
        plo = max(t0 - (K - 1) > 0 ? (t0 - (K - 1)) / stride : 0, 0);
        phi = min((t0 + 15) / stride, T - 1);
    } else {
        plo = t0 * stride - pad;
        phi = (t0 + 15) * stride + K - 1 - pad;
    }
    const int npos = max(phi - plo + 1, 0);
    const int cit = max(1, min(min(32, VQF_WS / (VQF_WP * K)), VQF_XS / max(npos, 1)));
    double acc[4];
    const double b0 = (bias && co < Cout) ? (double)bias[co] : 0.0;
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[j] = b0;
    const float *xb = x + (int64_t)b * T * Cin;
    for (int ci0 = 0; ci0 < Cin; ci0 += cit) {
        const int nci = min(cit, Cin - ci0);
        __syncthreads();
        if (TR) {   // W [Cin][Cout][K]: a chunk row (ci, k) runs over co with stride K
            for (int r = g; r < nci * K; r += 4) {
                const int ci = r / K, k = r - ci * K;
                ws[r * VQF_WP + col] = co < Cout ? W[((int64_t)(ci0 + ci) * Cout + co) * K + k] : 0.f;
            }
        } else {    // W [Cout][Cin][K]: each channel's chunk is nci K contiguous floats; read them in order
            const int run = nci * K;
            for (int e = tid; e < 64 * run; e += 256) {
                const int c = e / run, r = e - c * run;
                ws[r * VQF_WP + c] = co0 + c < Cout ? W[((int64_t)(co0 + c) * Cin + ci0) * K + r] : 0.f;
            }
        }
        if (S1K3) {   // window as [ci][pos]: a wave's taps of one channel are 6 consecutive doubles
            for (int e = tid; e < npos * nci; e += 256) {
                const int p = e / nci, ci = e - p * nci, pos = plo + p;
                xs[ci * npos + p] = (pos >= 0 && pos < T) ? (double)xb[(int64_t)pos * Cin + ci0 + ci] : 0.0;
            }
        } else {
            for (int e = tid; e < npos * nci; e += 256) {
                const int p = e / nci, ci = e - p * nci, pos = plo + p;
                xs[e] = (pos >= 0 && pos < T) ? (double)xb[(int64_t)pos * Cin + ci0 + ci] : 0.0;
            }
        }
        __syncthreads();
        if (S1K3) {
            // output 4 g + j, tap k reads window position 4 g + j + k
            for (int ci = 0; ci < nci; ++ci) {
                const double *xp = xs + ci * npos + 4 * g;
                double xv[6];
#pragma unroll
                for (int q = 0; q < 6; ++q) xv[q] = xp[q];
                const float *wp = ws + ci * 3 * VQF_WP + col;
#pragma unroll
                for (int k = 0; k < 3; ++k) {
                    const double w = (double)wp[k * VQF_WP];
#pragma unroll
                    for (int j = 0; j < 4; ++j) acc[j] += xv[j + k] * w;
                }
            }
        } else if (TR) {
            for (int ci = 0; ci < nci; ++ci)
                for (int k = 0; k < K; ++k) {
                    const double w = (double)ws[(ci * K + k) * VQF_WP + col];
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const int t = t0 + 4 * g + j, num = t - k;
                        const int ti = num / stride;
                        if (t < To && num >= 0 && num % stride == 0 && ti < T)
                            acc[j] += xs[(ti - plo) * nci + ci] * w;
                    }
                }
        } else {
            // output 4 g + j, tap k reads window position (4 g + j) stride + k
            const double *xc = xs + 4 * g * stride * nci;
            for (int ci = 0; ci < nci; ++ci) {
#pragma unroll
                for (int k = 0; k < K; ++k) {
                    const double w = (double)ws[(ci * K + k) * VQF_WP + col];
                    double xv[4];
#pragma unroll
                    for (int j = 0; j < 4; ++j) xv[j] = xc[(j * stride + k) * nci + ci];
#pragma unroll
                    for (int j = 0; j < 4; ++j) acc[j] += xv[j] * w;
                }
            }
        }
    }
    if (co < Cout) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int t = t0 + 4 * g + j;
            if (t >= To) continue;
            double v = acc[j];
            if (!TR && v == 0.0) v = vqf_conv_exact(xb, W, bias, T, Cin, co, K, stride, pad, t);
            y[((int64_t)b * To + t) * Cout + co] = (float)v;
        }
    }
}

// conv1d with kernel 3, stride 1, padding 1 and Cin % 32 == 0 (Phi and the
// refine convs): the layout and arithmetic of vqf_conv_body's S1K3 path, with
// the LDS sized to what it uses (5 workgroups per CU instead of 3) and
// division-free staging: a thread copies one contiguous 24-float run of one
// channel's weights; window entries map to threads by bits.
__device__ __forceinline__ void vqf_conv3_body(const float *__restrict__ x, const float *__restrict__ W,
                                               const float *__restrict__ bias, float *__restrict__ y, int T,
                                               int Cin, int Cout, int To) {
#pragma clang fp contract(off)
    __shared__ float ws[96 * VQF_WP];     // [ci * 3 + k][co], 32 input channels
    __shared__ double xs[32 * 18];        // [ci][pos], 18 window positions
    const int tid = threadIdx.x, col = tid & 63, g = tid >> 6;
    const int co0 = blockIdx.x * 64, t0 = blockIdx.y * 16, b = blockIdx.z;
    const int co = co0 + col, plo = t0 - 1;
    double acc[4];
    const double b0 = (bias && co < Cout) ? (double)bias[co] : 0.0;
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[j] = b0;
    const float *xb = x + (int64_t)b * T * Cin;
    const float *wrow = W + (int64_t)min(co, Cout - 1) * Cin * 3;   // this lane's channel (clamped; unused lanes write 0)
    for (int ci0 = 0; ci0 < Cin; ci0 += 32) {
        __syncthreads();
        {   // weights: lane col, rows 24 g .. 24 g + 23 of the chunk (one contiguous run)
            const float *src = wrow + ci0 * 3 + 24 * g;
#pragma unroll
            for (int i = 0; i < 24; ++i) ws[(24 * g + i) * VQF_WP + col] = co < Cout ? src[i] : 0.f;
        }
        {   // window: channel tid & 31, positions (tid >> 5) + 8 i
            const int ci = tid & 31;
#pragma unroll
            for (int i = 0; i < 3; ++i) {
                const int p = (tid >> 5) + 8 * i;
                if (p < 18) {
                    const int pos = plo + p;
                    xs[ci * 18 + p] = (pos >= 0 && pos < T) ? (double)xb[(int64_t)pos * Cin + ci0 + ci] : 0.0;
                }
            }
        }
        __syncthreads();
#pragma unroll 2
        for (int ci = 0; ci < 32; ++ci) {
            const double *xp = xs + ci * 18 + 4 * g;
            double xv[6];
#pragma unroll
            for (int q = 0; q < 6; ++q) xv[q] = xp[q];
            const float *wp = ws + ci * 3 * VQF_WP + col;
#pragma unroll
            for (int k = 0; k < 3; ++k) {
                const double w = (double)wp[k * VQF_WP];
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[j] += xv[j + k] * w;
            }
        }
    }
    if (co < Cout) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int t = t0 + 4 * g + j;
            if (t >= To) continue;
            double v = acc[j];
            if (v == 0.0) v = vqf_conv_exact(xb, W, bias, T, Cin, co, 3, 1, 1, t);
            y[((int64_t)b * To + t) * Cout + co] = (float)v;
        }
    }
}

extern "C" __global__ void __launch_bounds__(256)
vqf_conv3(const float *x, const float *W, const float *bias, float *y, int T, int Cin, int Cout, int K, int stride,
          int pad, int To) {
    vqf_conv3_body(x, W, bias, y, T, Cin, Cout, To);
}

extern "C" __global__ void __launch_bounds__(256)
vqf_conv1d(const float *x, const float *W, const float *bias, float *y, int T, int Cin, int Cout, int K, int stride,
           int pad, int To) {
    if (K == 3 && stride == 1) vqf_conv_body<false, 3, true>(x, W, bias, y, T, Cin, Cout, K, stride, pad, To);
    else vqf_conv_body<false, 0, false>(x, W, bias, y, T, Cin, Cout, K, stride, pad, To);
}

extern "C" __global__ void __launch_bounds__(256)
vqf_convT1d(const float *x, const float *W, const float *bias, float *y, int T, int Cin, int Cout, int K, int stride,
            int pad, int To) {
    vqf_conv_body<true, 0, false>(x, W, bias, y, T, Cin, Cout, K, stride, pad, To);
}

// kernels.c:618-640 GroupNorm (8 groups, no affine, eps 1e-5) of x [B][T][C]:
// one workgroup per (b, g); the fp64 mean and variance run serially in the
// reference's order (channel outer, position inner), then all threads
// normalise.
extern "C" __global__ void __launch_bounds__(64)
vqf_groupnorm(const float *__restrict__ x, float *__restrict__ y, int T, int C) {
#pragma clang fp contract(off)
    __shared__ double st[2];
    const int b = blockIdx.x >> 3, g = blockIdx.x & 7, Cg = C / 8;
    const float *xb = x + (int64_t)b * T * C + g * Cg;
    if (threadIdx.x == 0) {
        const int64_t cnt = (int64_t)Cg * T;
        double mean = 0.0;
        for (int c = 0; c < Cg; ++c)
            for (int t = 0; t < T; ++t) mean += (double)xb[(int64_t)t * C + c];
        mean /= (double)cnt;
        double var = 0.0;
        for (int c = 0; c < Cg; ++c)
            for (int t = 0; t < T; ++t) {
                const double d = (double)xb[(int64_t)t * C + c] - mean;
                var += d * d;
            }
        var /= (double)cnt;
        st[0] = mean;
        st[1] = 1.0 / sqrt(var + 1e-5);
    }
    __syncthreads();
    const double mean = st[0], inv = st[1];
    float *yb = y + (int64_t)b * T * C + g * Cg;
    for (int e = threadIdx.x; e < Cg * T; e += 64) {
        const int c = e % Cg, t = e / Cg;
        yb[(int64_t)t * C + c] = (float)(((double)xb[(int64_t)t * C + c] - mean) * inv);
    }
}

// vq.c:243-277 Phi blend h = (1 - r) h + r c (float); r == 0 adds: h += c
// (the refine step, vq.c:320-330)
extern "C" __global__ void __launch_bounds__(256)
vqf_blend(float *__restrict__ h, const float *__restrict__ c, int64_t n, float r, int add) {
#pragma clang fp contract(off)
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    h[i] = add ? h[i] + c[i] : (1.0f - r) * h[i] + r * c[i];
}

// q [B][tl][D] = codebook rows of level codes idx[b * total + off + t]
extern "C" __global__ void __launch_bounds__(256)
vqf_gather(const float *__restrict__ E, const int *__restrict__ idx, int V, int total, int off, int B, int tl, int D,
           float *__restrict__ q) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (int64_t)B * tl * D) return;
    const int d = (int)(i % D), r = (int)(i / D), b = r / tl, t = r - b * tl;
    int code = idx[(int64_t)b * total + off + t];
    if ((unsigned)code >= (unsigned)V) code = 0;
    q[i] = E[(int64_t)code * D + d];
}

// z_hat += up, z_rest -= up (vq.c:476-498); init: z_hat = 0 + up (the
// reference clears z_hat, then adds)
extern "C" __global__ void __launch_bounds__(256)
vqf_update(float *__restrict__ zh, float *__restrict__ zr, const float *__restrict__ up, int64_t n, int init) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    const float u = up[i];
    zh[i] = (init ? 0.0f : zh[i]) + u;
    if (zr) zr[i] = zr[i] - u;
}
