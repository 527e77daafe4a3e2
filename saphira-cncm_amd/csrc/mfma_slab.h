// mfma_slab.h -- operand slabs of 64 rows x 32 k for the FP32-MFMA kernels
// (v_mfma_f32_16x16x4_f32), loaded straight into LDS, and the fragment reads
// that feed the MFMAs.  Shared by the GEMMs and the VQ distance screen.
#pragma once
#include "ncm_dev.h"

#define GEMM_BK 32
#define GEMM_NT 256
#define OOB_OFFSET 0x80000000u

// Workgroups are dispatched round-robin over the 8 XCDs (each with its own
// L2): give every XCD a contiguous range of n work items.
__device__ __forceinline__ int xcd_remap(int j, int n) {
    return (n & 7) == 0 ? (j & 7) * (n >> 3) + (j >> 3) : j;
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const float *base, unsigned bytes) {
    return __builtin_amdgcn_make_buffer_rsrc((void *)base, (short)0, (int)bytes, 0x00020000);
}

// k-permutation: inside every 16-wide k chunk, MFMA step s (0..3) gives lane
// group g = lane/16 the reduction index k = 4g + s, for both operands; the
// MFMA sums over all 16 (g, s) pairs, so the product is unchanged and every
// k-contiguous fragment is one 128-bit LDS read.
//
// Kernels built on these slabs load them with buffer_load_dwordx4 ... lds:
// lane l of a load writes LDS bytes [16 l, 16 l + 16) after the wave's base
// (M0), from any global offset, so operands go from L2 to LDS without VGPR
// staging or LDS store instructions.  A slab is kept in its memory layout:
//   k-contiguous [64 rows][32 k]: pitch 32 floats, the float4 group g of k of
//     row r in slot g ^ (r & 7); fragment reads are one ds_read_b128 per
//     16-row block (see k-permutation below), conflict-free;
//   i/j-contiguous [32 k][64 cols]: pitch 64 floats, the float4 group c of
//     columns of k-row kr in slot c ^ (8 * ((kr >> 2) & 1)); the wave's MFMA
//     blocks b = 0, 1 take the interleaved columns 2 j + b, so one
//     ds_read_b64 at (kr, 2 j) feeds both blocks at one k; conflict-free.
#define D_SLAB (64 * GEMM_BK)   // floats per operand slab

template <bool KC>
struct DSlab {
    // The wave issues loads 2 * wave + e (e = 0, 1) of the slab's eight.
    unsigned voff[2];   // lane byte offset at k = 0; OOB_OFFSET outside the tile
    int klim[2];        // the lane's element is inside the k range iff slab k0 < klim
    __device__ __forceinline__ void init(int wave, int lane, int ld, int fix0, int fix_lim, int k_lim) {
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            const int q = 2 * wave + e;
            if (KC) {   // rows 8 q .. 8 q + 7, 8 lanes per row
                const int r = 8 * q + (lane >> 3), g = (lane & 7) ^ (r & 7);
                voff[e] = fix0 + r < fix_lim ? (unsigned)((fix0 + r) * ld + 4 * g) * 4u : OOB_OFFSET;
                klim[e] = k_lim - 4 * g;
            } else {    // k-rows 4 q .. 4 q + 3, 16 lanes per row
                const int kr = 4 * q + (lane >> 4), c = (lane & 15) ^ (8 * ((kr >> 2) & 1));
                voff[e] = fix0 + 4 * c < fix_lim ? (unsigned)(kr * ld + fix0 + 4 * c) * 4u : OOB_OFFSET;
                klim[e] = k_lim - kr;
            }
        }
    }
    __device__ __forceinline__ void load(__amdgpu_buffer_rsrc_t rs, float *slab, int wave, int k0, int ld) const {
        const unsigned dk = KC ? (unsigned)k0 * 4u : (unsigned)k0 * (unsigned)ld * 4u;
#pragma unroll
        for (int e = 0; e < 2; ++e)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                rs, (__attribute__((address_space(3))) void *)(slab + (2 * wave + e) * 256), 16,
                k0 < klim[e] ? voff[e] + dk : OOB_OFFSET, 0, 0, 0);
    }
};

// f[t][s]: the operand value of MFMA block t at step s of chunk kc, for the
// wave's 32 rows / columns starting at w * 32.
template <bool KC>
__device__ __forceinline__ void d_frags(const float *slab, int w, int li, int lg, int kc, float (&f)[2][4]) {
    if (KC) {
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            const int r = w * 32 + 16 * t + li;
            const f4 v = *(const f4 *)(slab + r * GEMM_BK + 4 * ((4 * kc + lg) ^ (r & 7)));
#pragma unroll
            for (int s = 0; s < 4; ++s) f[t][s] = v[s];
        }
    } else {
        const int col = w * 32 + 2 * li;
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            const int kr = 16 * kc + 4 * lg + s;
            const f2 v = *(const f2 *)(slab + kr * 64 + 4 * ((col >> 2) ^ (8 * (lg & 1))) + (col & 3));
            f[0][s] = v.x;
            f[1][s] = v.y;
        }
    }
}

// 128-row / 128-column slabs (the 128 x 128-tile GEMMs): k-contiguous [128 rows][32 k] as the 64-row slabs (pitch 32
// floats, float4 group g of row r in slot g ^ (r & 7)); i/j-contiguous [32
// k][128 cols] at pitch 128 with no swizzle: a wave's fragment read at
// (k-row kr, columns w*64 + 4 li .. + 3) is one ds_read_b128 that feeds its
// four MFMA blocks (block b takes column w*64 + 4 j + b), and the 16 lanes of
// a gfx950 ds_read_b128 service group -- {0-3, 12-15, 20-23, 24-27} or {4-7,
// 8-11, 16-19, 28-31}, lane = 16 lg + li -- then cover the 64 banks once
// (rows 4 lg apart start at bank 0, columns 4 li span 16 banks per lane
// quad).
#define BIG 128
#define D_SLAB_BIG (BIG * GEMM_BK)

template <bool KC>
struct DSlabBig {
    // The wave issues loads 4 * wave + e (e = 0..3) of the slab's sixteen.
    // k-contiguous: rows 8 q .. 8 q + 7 (8 lanes per row), a row bound per
    // load; i/j-contiguous: k-rows 2 q, 2 q + 1 (32 lanes per row), one column
    // bound for all four loads, which sit 2 e k-rows after load 0 (so only
    // load 0's offset and k bound are kept: registers are scarce here).
    unsigned voff[KC ? 4 : 1];
    int klim[KC ? 4 : 1];
    __device__ __forceinline__ void init(int wave, int lane, int ld, int fix0, int fix_lim, int k_lim) {
        if (KC) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int r = 8 * (4 * wave + e) + (lane >> 3), g = (lane & 7) ^ (r & 7);
                voff[e] = fix0 + r < fix_lim ? (unsigned)((fix0 + r) * ld + 4 * g) * 4u : OOB_OFFSET;
                klim[e] = k_lim - 4 * g;
            }
        } else {
            const int kr = 8 * wave + (lane >> 5), c = lane & 31;
            voff[0] = fix0 + 4 * c < fix_lim ? (unsigned)(kr * ld + fix0 + 4 * c) * 4u : OOB_OFFSET;
            klim[0] = k_lim - kr;
        }
    }
    __device__ __forceinline__ void load(__amdgpu_buffer_rsrc_t rs, float *slab, int wave, int k0, int ld) const {
        const unsigned dk = KC ? (unsigned)k0 * 4u : (unsigned)k0 * (unsigned)ld * 4u;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            unsigned off;
            if (KC)
                off = k0 < klim[e] ? voff[e] + dk : OOB_OFFSET;
            else   // an out-of-range column stays beyond the buffer after the k-row step
                off = k0 + 2 * e < klim[0] && voff[0] != OOB_OFFSET ? voff[0] + dk + (unsigned)(2 * e * ld) * 4u
                                                                   : OOB_OFFSET;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                rs, (__attribute__((address_space(3))) void *)(slab + (4 * wave + e) * 256), 16, off, 0, 0, 0);
        }
    }
};

// f[t][s]: the operand value of MFMA block t at step s of chunk kc, for the
// wave's 64 rows / columns starting at w * 64.
template <bool KC>
__device__ __forceinline__ void d_frags_big(const float *slab, int w, int li, int lg, int kc, float (&f)[4][4]) {
    if (KC) {
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const int r = w * 64 + 16 * t + li;
            const f4 v = *(const f4 *)(slab + r * GEMM_BK + 4 * ((4 * kc + lg) ^ (r & 7)));
#pragma unroll
            for (int s = 0; s < 4; ++s) f[t][s] = v[s];
        }
    } else {
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            const int kr = 16 * kc + 4 * lg + s;
            const f4 v = *(const f4 *)(slab + kr * BIG + w * 64 + 4 * li);
#pragma unroll
            for (int t = 0; t < 4; ++t) f[t][s] = v[t];
        }
    }
}

