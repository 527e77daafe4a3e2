// ncm_dev.h -- device helpers shared by the gfx950 kernels of libncmhip.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

typedef float f4 __attribute__((ext_vector_type(4)));
typedef float f2 __attribute__((ext_vector_type(2)));

// Activation codes; must match NCM_ACT_* in include/ncm_hip.h.
enum { ACT_NONE = 0, ACT_SILU = 1, ACT_GELU = 2, ACT_GELU_TANH = 3, ACT_RELU2 = 4 };

// tanh in fp64 as 1 - 2 / (e^(2|t|) + 1) with the sign of t: absolute error
// within a few units of 2^-53 (the quantity the GELU forms use, inside
// 1 + tanh and 1 - tanh^2), at about a third of the instructions of the
// library's compensated tanh; e^(2|t|) = inf gives exactly 1.
__device__ __forceinline__ double ncm_tanh_d(double t) {
#pragma clang fp contract(off)
    const double e = exp(2.0 * fabs(t));
    return copysign(1.0 - 2.0 / (e + 1.0), t);
}

// Activations in the form the reference applies them to a float value
// (kernels.c:167-174 SiLU/GELU in float; kernels.c:207-218 gelu_new, whose
// CPU path evaluates in double).
__device__ __forceinline__ float ncm_act(float v, int act) {
    switch (act) {
    case ACT_SILU: return v / (1.0f + expf(-v));
    case ACT_GELU: return 0.5f * v * (1.0f + erff(v * 0.7071067811865475f));
    case ACT_GELU_TANH: {
        double d = v;
        double t = 0.7978845608028654 * (d + 0.044715 * d * d * d);
        return (float)(0.5 * d * (1.0 + ncm_tanh_d(t)));
    }
    case ACT_RELU2: {   // ncp.c:327-333: r = v > 0 ? v : 0; r * r (NaN -> 0)
        const float r = v > 0.f ? v : 0.f;
        return r * r;
    }
    default: return v;
    }
}

// dy * act'(x) in fp64, rounded to float (the reference's activation
// backward): kind 0 GELU (erf), 1 SiLU, 2 GELU (tanh form)
__device__ __forceinline__ float act_bwd_one(float xf, float dyf, int kind) {
#pragma clang fp contract(off)
    const double xv = (double)xf;
    double g;
    if (kind == 0) {
        const double e = erf(xv / 1.4142135623730951);
        g = 0.5 * (1 + e) + xv * exp(-0.5 * xv * xv) * 0.3989422804014327;
    } else if (kind == 1) {
        const double s = 1.0 / (1.0 + exp(-xv));
        g = s * (1 + xv * (1 - s));
    } else {
        const double c0 = 0.7978845608028654, c1 = 0.044715;
        const double th = ncm_tanh_d(c0 * (xv + c1 * xv * xv * xv));
        g = 0.5 * (1.0 + th) + 0.5 * xv * (1.0 - th * th) * c0 * (1.0 + 3.0 * c1 * xv * xv);
    }
    return (float)((double)dyf * g);
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

__device__ __forceinline__ double wave_sum_d(double v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

// Column swizzle of the SDPA kernels' 64 x 64 LDS tiles (row pitch 72
// floats): float column c of row r is stored at c ^ 16 when bits 2 and 3 of r
// differ.  Both fragment reads of those kernels -- lane (li, g) reading row
// 16c + li at columns 16kc + 4g, and reading row 16c + 4g + s at columns 4li
// -- then touch 64 distinct banks in every group of 16 lanes that
// ds_read_b128 serves per cycle on gfx950 ({0-3, 12-15, 20-23, 24-27},
// {4-7, 8-11, 16-19, 28-31} and the same + 32); unswizzled, the second read
// was 2-way conflicted.
#define LDS_SWZ(r, c) ((c) ^ (((((r) >> 2) ^ ((r) >> 3)) & 1) << 4))

// One 16x16x4 fp32 MFMA: lane l supplies A[l%16][l/16] and B[l/16][l%16];
// the result holds D[4*(l/16)+r][l%16] in component r.
__device__ __forceinline__ f4 mfma4(float a, float b, f4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

template <int ROWS, int COLS, int NT, bool VEC>
struct TileLoader {
    static constexpr int F4 = ROWS * COLS / 4;
    static constexpr int PER = (F4 + NT - 1) / NT;
    f4 r[PER];

    // Loads the ROWS x COLS tile whose top-left element is src[row0*ld + col0];
    // rows >= row_end or cols >= col_end read as zero.
    __device__ __forceinline__ void load(const float *__restrict__ src, int ld, int row0, int col0,
                                         int row_end, int col_end, int tid) {
#pragma unroll
        for (int j = 0; j < PER; ++j) {
            int f = tid + j * NT;
            int rr = f / (COLS / 4);
            int cc = (f % (COLS / 4)) * 4;
            int gr = row0 + rr, gc = col0 + cc;
            f4 v = {0.f, 0.f, 0.f, 0.f};
            if ((F4 % NT == 0 || f < F4) && gr < row_end) {
                const float *p = src + (int64_t)gr * ld + gc;
                if (VEC) {
                    if (gc < col_end) v = *(const f4 *)p;
                } else {
                    if (gc + 0 < col_end) v.x = p[0];
                    if (gc + 1 < col_end) v.y = p[1];
                    if (gc + 2 < col_end) v.z = p[2];
                    if (gc + 3 < col_end) v.w = p[3];
                }
            }
            r[j] = v;
        }
    }

    __device__ __forceinline__ void store(float *dst, int tid) {
        constexpr int LD = COLS + 4;
#pragma unroll
        for (int j = 0; j < PER; ++j) {
            int f = tid + j * NT;
            if (F4 % NT == 0 || f < F4) {
                int rr = f / (COLS / 4);
                int cc = (f % (COLS / 4)) * 4;
                *(f4 *)(dst + rr * LD + cc) = r[j];
            }
        }
    }
};

