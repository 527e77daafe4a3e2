// gemm.hip -- FP32 MFMA GEMMs (gfx950, v_mfma_f32_16x16x4_f32) behind the
// linear forward and backward of cncm.
//
// One kernel template computes C[i,j] (i < Mo, j < No) = sum_k A(i,k) B(k,j)
// for the three operand layouts the linear layer needs (all row-major fp32):
//
//   forward  y  = x . W^T : A(i,k) = x[i*K+k]   (k-contiguous, "AKC")
//                          B(k,j) = W[j*K+k]   (k-contiguous, "BKC")
//   dX       dx = dy . W  : A(i,k) = dy[i*M+k]  (k-contiguous)
//                          B(k,j) = W[k*K+j]   (j-contiguous)
//   dW       dW = dy^T. x : A(i,k) = dy[k*M+i]  (i-contiguous)
//                          B(k,j) = x[k*K+j]   (j-contiguous)
//
// Tiling: a 256-thread workgroup owns a 64x64 output tile; each of its four
// 64-lane waves owns a 32x32 sub-tile of 2x2 MFMA blocks.  Operand slabs of
// BK = 32 go global -> registers -> LDS (two buffers) and are consumed as two
// 16-wide chunks; the small register (~90 VGPRs) and LDS (36 KB) footprint
// lets four workgroups share a CU, whose interleaving hides the load and
// barrier latency.  Both operands are kept k-contiguous in LDS: a slab whose
// memory layout is i/j-contiguous is transposed by its LDS store.  Global
// loads are raw buffer loads: lanes outside the matrix get an offset beyond
// the buffer and read zero, so the loop body has no branches.
//
// k-permutation: inside every 16-wide chunk, MFMA step s (0..3) gives lane
// group g = lane/16 the reduction index k = 4g + s, for both operands.  The
// MFMA sums over all 16 (g, s) pairs, so the product is unchanged, but every
// operand fragment becomes one 128-bit LDS read (a float4 along k covers the
// 4 steps).
//
// Scheduling: tiles [0, dp_tiles) run whole, one workgroup each; every other
// tile is cut into `segs` k-segments that fill the last round of the chip.
// Segments store partial tiles; gemm64_fixup (a second launch) sums them in
// segment order -- deterministic -- and applies the epilogue.
//
// Accuracy: MFMAs accumulate 128 k into `acc`, which is then added into `tot`;
// a single fp32 chain over K terms has an error growing like K u, the two
// levels keep it near (128 + K/128) u.
//
// Epilogues: STORE  C = res + act(acc + bias);  ACCUM  C += acc.
#include "ncm_dev.h"

enum { EPI_STORE = 0, EPI_ACCUM = 1 };

struct GemmArgs {
    const float *A;
    const float *B;
    float *C;
    const float *bias;   // [No] or null (STORE only)
    const float *res;    // [Mo, ldc] or null (STORE only)
    float *ws;           // partial tiles of split tiles [units][64*64]
    int Mo, No, K;
    int lda, ldb, ldc;
    int act;
    int vec_out;         // unused by the 64x64 kernels (kept for the host's struct layout)
    int tiles_m, tiles_n;
    int iters;           // BK slabs per tile (a multiple of 4)
    int dp_tiles;        // blocks [0, dp_tiles): one whole tile each
    int segs;            // later blocks: k-segment (u % segs) of tile dp_tiles + u / segs
    unsigned a_bytes, b_bytes;  // extents of A and B for the buffer descriptors
};

#define GEMM_BK 32
#define GEMM_NT 256
#define OOB_OFFSET 0x80000000u

// Grouped raster: GROUP_M tile rows advance together along N so that the B
// panels they share stay in L2.
template <int GROUP_M>
__device__ __forceinline__ void tile_rc(int t, int tiles_m, int tiles_n, int &tm, int &tn) {
    int group = GROUP_M * tiles_n;
    int g = t / group;
    int first = g * GROUP_M;
    int gm = min(tiles_m - first, GROUP_M);
    int in = t - g * group;
    tm = first + in % gm;
    tn = in / gm;
}

// Workgroups are dispatched round-robin over the 8 XCDs (each with its own
// L2): give every XCD a contiguous range of n work items.
__device__ __forceinline__ int xcd_remap(int j, int n) {
    return (n & 7) == 0 ? (j & 7) * (n >> 3) + (j >> 3) : j;
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const float *base, unsigned bytes) {
    return __builtin_amdgcn_make_buffer_rsrc((void *)base, (short)0, (int)bytes, 0x00020000);
}

// db[m] += (float) sum_r dy[r,m], the bias gradient of train_tape.c:708-713,
// accumulated in fp64 as there.  Stage 1 (COLSUM_ROWS rows per chunk):
// lane = 4 columns (float4), the 4 waves take interleaved rows, an LDS
// reduction combines them; stage 2 sums the chunk partials in order.
#define COLSUM_ROWS 64
extern "C" __global__ void __launch_bounds__(256)
colsum_partial_v(const float *__restrict__ dy, int64_t rows, int N, double *__restrict__ part) {
    __shared__ double red[3][64][4];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int col = (blockIdx.x * 64 + lane) * 4;
    const int64_t r0 = (int64_t)blockIdx.y * COLSUM_ROWS;
    const int64_t r1 = min(rows, r0 + COLSUM_ROWS);
    double s0 = 0.0, s1 = 0.0, s2 = 0.0, s3 = 0.0;
    if (col < N) {
#pragma unroll 4
        for (int64_t r = r0 + wave; r < r1; r += 4) {
            f4 v = *(const f4 *)(dy + r * N + col);
            s0 += v.x; s1 += v.y; s2 += v.z; s3 += v.w;
        }
    }
    if (wave > 0) {
        red[wave - 1][lane][0] = s0; red[wave - 1][lane][1] = s1;
        red[wave - 1][lane][2] = s2; red[wave - 1][lane][3] = s3;
    }
    __syncthreads();
    if (wave == 0 && col < N) {
        for (int w = 0; w < 3; ++w) {
            s0 += red[w][lane][0]; s1 += red[w][lane][1]; s2 += red[w][lane][2]; s3 += red[w][lane][3];
        }
        double *o = part + (int64_t)blockIdx.y * N + col;
        o[0] = s0; o[1] = s1; o[2] = s2; o[3] = s3;
    }
}

extern "C" __global__ void __launch_bounds__(256)
colsum_partial_s(const float *__restrict__ dy, int64_t rows, int N, double *__restrict__ part) {
    int col = blockIdx.x * 256 + threadIdx.x;
    if (col >= N) return;
    int64_t r0 = (int64_t)blockIdx.y * COLSUM_ROWS;
    int64_t r1 = min(rows, r0 + COLSUM_ROWS);
    double s = 0.0;
    for (int64_t r = r0; r < r1; ++r) s += (double)dy[r * N + col];
    part[(int64_t)blockIdx.y * N + col] = s;
}

extern "C" __global__ void __launch_bounds__(256)
colsum_final(const double *__restrict__ part, int chunks, int N, float *db) {
    int col = blockIdx.x * 256 + threadIdx.x;
    if (col >= N) return;
    double s = 0.0;
#pragma unroll 16
    for (int c = 0; c < chunks; ++c) s += part[(int64_t)c * N + col];
    db[col] += (float)s;
}

// ---- small-batch backward (batch <= 8 rows of dy) ----
// dW[n,k] += sum_r dy[r,n] x[r,k]: the reference's per-output fp64 sum over
// r ascending, rounded to float and added through a zeroed temporary
// (train_tape.c:714-720), so this path is bit-exact with the host backward.
// One thread per 4 consecutive k of one row n; HBM-bound on dW.
template <bool VEC>
__device__ __forceinline__ void dw_rank_body(const float *__restrict__ dy, const float *__restrict__ x,
                                             float *dW, int nb, int N, int K) {
#pragma clang fp contract(off)
    const int64_t f = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int K4 = (K + 3) / 4;
    if (f >= (int64_t)N * K4) return;
    const int n = (int)(f / K4), k = (int)(f % K4) * 4;
    double s[4] = {0.0, 0.0, 0.0, 0.0};
    for (int r = 0; r < nb; ++r) {
        const double g = dy[(int64_t)r * N + n];
        const float *xr = x + (int64_t)r * K + k;
        if (VEC) {
            f4 v = *(const f4 *)xr;
            s[0] += g * v.x; s[1] += g * v.y; s[2] += g * v.z; s[3] += g * v.w;
        } else {
#pragma unroll
            for (int u = 0; u < 4; ++u) if (k + u < K) s[u] += g * xr[u];
        }
    }
    float *o = dW + (int64_t)n * K + k;
    if (VEC) {
        f4 w = *(f4 *)o;
        w.x += 0.0f + (float)s[0]; w.y += 0.0f + (float)s[1];
        w.z += 0.0f + (float)s[2]; w.w += 0.0f + (float)s[3];
        *(f4 *)o = w;
    } else {
#pragma unroll
        for (int u = 0; u < 4; ++u) if (k + u < K) o[u] += 0.0f + (float)s[u];
    }
}

extern "C" __global__ void __launch_bounds__(256)
dw_rank_v(const float *dy, const float *x, float *dW, int nb, int N, int K) { dw_rank_body<true>(dy, x, dW, nb, N, K); }
extern "C" __global__ void __launch_bounds__(256)
dw_rank_s(const float *dy, const float *x, float *dW, int nb, int N, int K) { dw_rank_body<false>(dy, x, dW, nb, N, K); }

// dx[r,k] += sum_n dy[r,n] W[n,k] for r < nb: a transposed GEMV streaming W
// once.  Block = 4 waves x 256 columns (float4 per lane); the waves take
// interleaved rows n of a chunk of DXT_ROWS rows, LDS combines them, and the
// chunk partials [chunk][nb][K] are summed in chunk order by dxt_final.
#define DXT_ROWS 32
template <int NB>
__device__ __forceinline__ void dxt_partial_body(const float *__restrict__ dy, const float *__restrict__ W,
                                                 int N, int K, float *__restrict__ part) {
    __shared__ f4 red[3][NB][64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int col = (blockIdx.x * 64 + lane) * 4;
    const int n0 = blockIdx.y * DXT_ROWS, n1 = min(N, n0 + DXT_ROWS);
    f4 acc[NB];
#pragma unroll
    for (int b = 0; b < NB; ++b) acc[b] = f4{0.f, 0.f, 0.f, 0.f};
    if (col < K) {
#pragma unroll 4
        for (int n = n0 + wave; n < n1; n += 4) {
            f4 w = __builtin_nontemporal_load((const f4 *)(W + (int64_t)n * K + col));
#pragma unroll
            for (int b = 0; b < NB; ++b) acc[b] += dy[(int64_t)b * N + n] * w;
        }
    }
    if (wave > 0) {
#pragma unroll
        for (int b = 0; b < NB; ++b) red[wave - 1][b][lane] = acc[b];
    }
    __syncthreads();
    if (wave == 0 && col < K) {
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            f4 v = acc[b] + red[0][b][lane] + red[1][b][lane] + red[2][b][lane];
            *(f4 *)(part + ((int64_t)blockIdx.y * NB + b) * K + col) = v;
        }
    }
}

extern "C" __global__ void __launch_bounds__(256)
dxt_final(const float *__restrict__ part, int chunks, int nb, int K, float *__restrict__ dx) {
    int64_t f = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (f >= (int64_t)nb * K) return;
    float s = 0.f;
#pragma unroll 16
    for (int c = 0; c < chunks; ++c) s += part[(int64_t)c * nb * K + f];
    dx[f] += s;
}

#define DXT_KERNEL(NB) \
    extern "C" __global__ void __launch_bounds__(256) \
    dxt_partial_b##NB(const float *dy, const float *W, int N, int K, float *part) { dxt_partial_body<NB>(dy, W, N, K, part); }
DXT_KERNEL(1)
DXT_KERNEL(2)
DXT_KERNEL(4)
DXT_KERNEL(8)

// ---- GEMV: y[b,n] = res + act(bias[n] + sum_k x[b,k] W[n,k]) for NB <= 8
// batch rows (decode).  HBM-bound on W: each workgroup streams R rows of W
// with 128-bit loads, unrolled 4 deep to keep loads in flight, and reuses
// every x chunk across its R rows.
struct GemvArgs {
    const float *x;
    const float *W;
    const float *bias;
    const float *res;
    float *y;
    int N, K;
    int act;
};

template <int NB, int R, bool VEC>
__device__ __forceinline__ void gemv_body(const GemvArgs &p) {
    const int tid = threadIdx.x;
    const int n0 = blockIdx.x * R;
    float acc[R][NB];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int b = 0; b < NB; ++b) acc[r][b] = 0.f;

    const float *wr[R];
#pragma unroll
    for (int r = 0; r < R; ++r) wr[r] = p.W + (int64_t)min(n0 + r, p.N - 1) * p.K;

    if (VEC) {
        const int K4 = p.K >> 2;
        int c = tid;
        for (; c + 3 * 256 < K4; c += 4 * 256) {
            f4 w[4][R];
#pragma unroll
            for (int u = 0; u < 4; ++u)
#pragma unroll
                for (int r = 0; r < R; ++r)
                    w[u][r] = __builtin_nontemporal_load((const f4 *)wr[r] + c + u * 256);
#pragma unroll
            for (int u = 0; u < 4; ++u) {
#pragma unroll
                for (int b = 0; b < NB; ++b) {
                    f4 xv = *((const f4 *)(p.x + (int64_t)b * p.K) + c + u * 256);
#pragma unroll
                    for (int r = 0; r < R; ++r)
                        acc[r][b] += w[u][r].x * xv.x + w[u][r].y * xv.y + w[u][r].z * xv.z + w[u][r].w * xv.w;
                }
            }
        }
        for (; c < K4; c += 256) {
            f4 w[R];
#pragma unroll
            for (int r = 0; r < R; ++r) w[r] = __builtin_nontemporal_load((const f4 *)wr[r] + c);
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                f4 xv = *((const f4 *)(p.x + (int64_t)b * p.K) + c);
#pragma unroll
                for (int r = 0; r < R; ++r)
                    acc[r][b] += w[r].x * xv.x + w[r].y * xv.y + w[r].z * xv.z + w[r].w * xv.w;
            }
        }
    } else {
        for (int k = tid; k < p.K; k += 256) {
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                float xv = p.x[(int64_t)b * p.K + k];
#pragma unroll
                for (int r = 0; r < R; ++r) acc[r][b] += wr[r][k] * xv;
            }
        }
    }

    __shared__ float red[4][R * NB];
    const int lane = tid & 63, wave = tid >> 6;
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            float v = wave_sum(acc[r][b]);
            if (lane == 0) red[wave][r * NB + b] = v;
        }
    __syncthreads();
    if (tid < R * NB) {
        int r = tid / NB, b = tid % NB;
        int n = n0 + r;
        if (n < p.N) {
            float v = (red[0][tid] + red[1][tid]) + (red[2][tid] + red[3][tid]);
            if (p.bias) v += p.bias[n];
            v = ncm_act(v, p.act);
            if (p.res) v = p.res[(int64_t)b * p.N + n] + v;
            p.y[(int64_t)b * p.N + n] = v;
        }
    }
}

// ---- instantiations (extern "C" names are looked up by the host runtime) ----
#define GEMV_KERNEL(name, NB, R, VEC) \
    extern "C" __global__ void __launch_bounds__(256) name(GemvArgs p) { gemv_body<NB, R, VEC>(p); }

GEMV_KERNEL(gemv_b1_r1_v, 1, 1, true)
GEMV_KERNEL(gemv_b1_r2_v, 1, 2, true)
GEMV_KERNEL(gemv_b1_r4_v, 1, 4, true)
GEMV_KERNEL(gemv_b2_r2_v, 2, 2, true)
GEMV_KERNEL(gemv_b4_r2_v, 4, 2, true)
GEMV_KERNEL(gemv_b8_r1_v, 8, 1, true)
GEMV_KERNEL(gemv_b1_r1_s, 1, 1, false)
GEMV_KERNEL(gemv_b2_r1_s, 2, 1, false)
GEMV_KERNEL(gemv_b4_r1_s, 4, 1, false)
GEMV_KERNEL(gemv_b8_r1_s, 8, 1, false)

// ---------------------------------------------------------------- GEMM (64x64 tiles)
// Per slab: store the slab loaded in the previous iteration to the free LDS
// buffer, issue the loads of the slab after it, run the 32 MFMAs of the
// current buffer, barrier.  The 36-float LDS pitch makes the fragment reads
// conflict-free.
#define G64 64
#define G64_LD (GEMM_BK + 4)
// LDS element (row, k) of a slab lives at row * G64_LD + swz(row, k): the
// float4 group of k is XORed with (row >> 4) & 3.  Fragment reads (16
// consecutive rows, one float4 each) keep a constant XOR and stay one aligned
// float4; the transposing stores of an i/j-contiguous slab (rows 4c + u,
// c = 0..15) then fall on 64 distinct banks instead of 16.
__device__ __forceinline__ int g64_swz(int row, int k) { return ((((k >> 2) ^ (row >> 4)) & 7) << 2) | (k & 3); }

template <bool KC, bool VEC>
struct Slab64 {
    // KC: memory [64 rows][K] (k along columns); else memory [K][64 cols]
    f4 r[2];
    int a0, b0;   // KC: row (t >> 3) + {0, 32}, k (t & 7) * 4;  !KC: k (t >> 4) + {0, 16}, i (t & 15) * 4
    __device__ __forceinline__ void init(int tid) {
        if (KC) { a0 = tid >> 3; b0 = (tid & 7) * 4; }
        else { a0 = tid >> 4; b0 = (tid & 15) * 4; }
    }
    // fix0: first row (KC) / column (!KC) of the tile; k0: first k of the slab
    __device__ __forceinline__ void load(__amdgpu_buffer_rsrc_t rs, int ld, int fix0, int k0, int fix_lim,
                                         int k_lim) {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int rw = KC ? fix0 + a0 + 32 * j : k0 + a0 + 16 * j;
            const int cl = KC ? k0 + b0 : fix0 + b0;
            const bool in_r = KC ? rw < fix_lim : rw < k_lim;
            const int lim_c = KC ? k_lim : fix_lim;
            const unsigned o = (unsigned)(rw * ld + cl) * 4u;
            if (VEC) {
                r[j] = __builtin_bit_cast(
                    f4, __builtin_amdgcn_raw_buffer_load_b128(rs, (in_r && cl < lim_c) ? o : OOB_OFFSET, 0, 0));
            } else {
#pragma unroll
                for (int u = 0; u < 4; ++u)
                    r[j][u] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                                            rs, (in_r && cl + u < lim_c) ? o + 4u * u : OOB_OFFSET, 0, 0));
            }
        }
    }
    __device__ __forceinline__ void store(float *buf) const {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            if (KC) {
                const int row = a0 + 32 * j;
                *(f4 *)(buf + row * G64_LD + g64_swz(row, b0)) = r[j];
            } else {
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    const int row = b0 + u;
                    buf[row * G64_LD + g64_swz(row, a0 + 16 * j)] = r[j][u];
                }
            }
        }
    }
};

template <int ACT, int EPI>
__device__ __forceinline__ void g64_out(const GemmArgs &p, int i, int j, float v) {
    if (i >= p.Mo || j >= p.No) return;
    float *c = p.C + (int64_t)i * p.ldc + j;
    if (EPI == EPI_ACCUM) {
        *c = *c + v;
    } else {
        if (p.bias) v += p.bias[j];
        v = ncm_act(v, ACT);
        if (p.res) v = p.res[(int64_t)i * p.ldc + j] + v;
        *c = v;
    }
}

// tot[a][b][r]: row wm*32 + a*16 + 4*lg + r, column wn*32 + b*16 + li
template <int EPI, int ACT>
__device__ __forceinline__ void g64_epilogue_act(const GemmArgs &p, const f4 (&tot)[2][2], int i0, int j0, int tid) {
    const int lane = tid & 63, wave = tid >> 6, wm = wave >> 1, wn = wave & 1;
    const int li = lane & 15, lg = lane >> 4;
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int b = 0; b < 2; ++b)
#pragma unroll
            for (int r = 0; r < 4; ++r)
                g64_out<ACT, EPI>(p, i0 + wm * 32 + a * 16 + 4 * lg + r, j0 + wn * 32 + b * 16 + li, tot[a][b][r]);
}

template <int EPI>
__device__ __forceinline__ void g64_epilogue(const GemmArgs &p, const f4 (&tot)[2][2], int i0, int j0, int tid) {
    if (EPI == EPI_ACCUM) { g64_epilogue_act<EPI, ACT_NONE>(p, tot, i0, j0, tid); return; }
    switch (p.act) {
    case ACT_SILU: g64_epilogue_act<EPI, ACT_SILU>(p, tot, i0, j0, tid); break;
    case ACT_GELU: g64_epilogue_act<EPI, ACT_GELU>(p, tot, i0, j0, tid); break;
    case ACT_GELU_TANH: g64_epilogue_act<EPI, ACT_GELU_TANH>(p, tot, i0, j0, tid); break;
    default: g64_epilogue_act<EPI, ACT_NONE>(p, tot, i0, j0, tid); break;
    }
}

template <bool AKC, bool BKC, int EPI, bool VEC>
__device__ __forceinline__ void gemm64_body(const GemmArgs &p) {
    __shared__ __attribute__((aligned(16))) float sA[2 * G64 * G64_LD];
    __shared__ __attribute__((aligned(16))) float sB[2 * G64 * G64_LD];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1, li = lane & 15, lg = lane >> 4;

    int tile, it0, it1, unit = -1;
    {
        const int b = blockIdx.x;
        if (b < p.dp_tiles) {
            tile = xcd_remap(b, p.dp_tiles);
            it0 = 0;
            it1 = p.iters;
        } else {
            const int ntail = (p.tiles_m * p.tiles_n - p.dp_tiles) * p.segs;
            const int j = b - p.dp_tiles;
            unit = ((p.dp_tiles & 7) == 0) ? xcd_remap(j, ntail) : j;
            const int tail = unit / p.segs, seg = unit - tail * p.segs;
            tile = p.dp_tiles + tail;
            const int q4 = p.iters >> 2;
            it0 = (int)((int64_t)seg * q4 / p.segs) * 4;
            it1 = (int)((int64_t)(seg + 1) * q4 / p.segs) * 4;
        }
    }
    int tm, tn;
    tile_rc<8>(tile, p.tiles_m, p.tiles_n, tm, tn);
    const int i0 = tm * G64, j0 = tn * G64;
    const int kend = min(p.K, it1 * GEMM_BK);
    const __amdgpu_buffer_rsrc_t ra = make_rsrc(p.A, p.a_bytes), rb = make_rsrc(p.B, p.b_bytes);
    Slab64<AKC, VEC> la;
    Slab64<BKC, VEC> lb;
    la.init(tid);
    lb.init(tid);

    f4 acc[2][2], tot[2][2];
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int b = 0; b < 2; ++b) acc[a][b] = tot[a][b] = f4{0.f, 0.f, 0.f, 0.f};

    auto chunk = [&](const float *a_s, const float *b_s, int kc) {
        f4 fa[2], fb[2];
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            const int ra_ = wm * 32 + t * 16 + li, rb_ = wn * 32 + t * 16 + li;
            fa[t] = *(const f4 *)(a_s + ra_ * G64_LD + g64_swz(ra_, kc * 16 + 4 * lg));
            fb[t] = *(const f4 *)(b_s + rb_ * G64_LD + g64_swz(rb_, kc * 16 + 4 * lg));
        }
#pragma unroll
        for (int s = 0; s < 4; ++s)
#pragma unroll
            for (int a = 0; a < 2; ++a)
#pragma unroll
                for (int b = 0; b < 2; ++b) acc[a][b] = mfma4(fa[a][s], fb[b][s], acc[a][b]);
    };

    la.load(ra, p.lda, i0, it0 * GEMM_BK, p.Mo, kend);
    lb.load(rb, p.ldb, j0, it0 * GEMM_BK, p.No, kend);
    la.store(sA);
    lb.store(sB);
    la.load(ra, p.lda, i0, (it0 + 1) * GEMM_BK, p.Mo, kend);
    lb.load(rb, p.ldb, j0, (it0 + 1) * GEMM_BK, p.No, kend);
    __syncthreads();
    for (int kt = it0; kt < it1; kt += 4) {
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int cur = u & 1;   // it0 is a multiple of 4: slab kt+u lives in buffer u & 1
            la.store(sA + (cur ^ 1) * G64 * G64_LD);
            lb.store(sB + (cur ^ 1) * G64 * G64_LD);
            la.load(ra, p.lda, i0, (kt + u + 2) * GEMM_BK, p.Mo, kend);
            lb.load(rb, p.ldb, j0, (kt + u + 2) * GEMM_BK, p.No, kend);
            chunk(sA + cur * G64 * G64_LD, sB + cur * G64 * G64_LD, 0);
            chunk(sA + cur * G64 * G64_LD, sB + cur * G64 * G64_LD, 1);
            __syncthreads();
        }
#pragma unroll
        for (int a = 0; a < 2; ++a)
#pragma unroll
            for (int b = 0; b < 2; ++b) {
                tot[a][b] += acc[a][b];
                acc[a][b] = f4{0.f, 0.f, 0.f, 0.f};
            }
    }
    if (unit >= 0) {
        float *mine = p.ws + (int64_t)unit * (G64 * G64);
#pragma unroll
        for (int a = 0; a < 2; ++a)
#pragma unroll
            for (int b = 0; b < 2; ++b) *(f4 *)(mine + ((a * 2 + b) * GEMM_NT + tid) * 4) = tot[a][b];
        return;
    }
    g64_epilogue<EPI>(p, tot, i0, j0, tid);
}

// Sum of the segment partials of split tile blockIdx.x in segment order, then
// the epilogue.
template <int EPI>
__device__ __forceinline__ void gemm64_fixup_body(const GemmArgs &p) {
    const int tid = threadIdx.x, tail = blockIdx.x;
    int tm, tn;
    tile_rc<8>(p.dp_tiles + tail, p.tiles_m, p.tiles_n, tm, tn);
    const float *first = p.ws + (int64_t)tail * p.segs * (G64 * G64);
    f4 tot[2][2];
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int b = 0; b < 2; ++b) tot[a][b] = *(const f4 *)(first + ((a * 2 + b) * GEMM_NT + tid) * 4);
    for (int s = 1; s < p.segs; ++s) {
        const float *part = first + (int64_t)s * (G64 * G64);
#pragma unroll
        for (int a = 0; a < 2; ++a)
#pragma unroll
            for (int b = 0; b < 2; ++b) tot[a][b] += *(const f4 *)(part + ((a * 2 + b) * GEMM_NT + tid) * 4);
    }
    g64_epilogue<EPI>(p, tot, tm * G64, tn * G64, tid);
}

#define GEMM64_KERNEL(name, AKC, BKC, EPI, VEC) \
    extern "C" __global__ void __launch_bounds__(GEMM_NT) name(GemmArgs p) { gemm64_body<AKC, BKC, EPI, VEC>(p); }
#define GEMM64_FIXUP(name, EPI) \
    extern "C" __global__ void __launch_bounds__(GEMM_NT) name(GemmArgs p) { gemm64_fixup_body<EPI>(p); }
GEMM64_KERNEL(gemm64_fwd_v, true,  true,  EPI_STORE, true)
GEMM64_KERNEL(gemm64_fwd_s, true,  true,  EPI_STORE, false)
GEMM64_KERNEL(gemm64_dx_v,  true,  false, EPI_ACCUM, true)
GEMM64_KERNEL(gemm64_dx_s,  true,  false, EPI_ACCUM, false)
GEMM64_KERNEL(gemm64_dw_v,  false, false, EPI_ACCUM, true)
GEMM64_KERNEL(gemm64_dw_s,  false, false, EPI_ACCUM, false)
GEMM64_FIXUP(gemm64_fixup_store, EPI_STORE)
GEMM64_FIXUP(gemm64_fixup_accum, EPI_ACCUM)
