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
// A workgroup owns a BM x BN output tile; each of its 64-lane waves owns a
// WM x WN sub-tile made of 16x16 MFMA blocks.  Operand tiles are staged
// global -> registers -> LDS with two LDS buffers, so the global loads for
// slab k+1 are in flight while slab k feeds the matrix cores.
//
// k-permutation: inside every 16-wide k chunk, MFMA step s (0..3) gives lane
// group g = lane/16 the reduction index k = 4g + s, for both operands.  The
// MFMA sums over all 16 (g, s) pairs, so the product is unchanged, but the
// operand reads become 128-bit LDS loads:
//   k-contiguous operand : one float4 along k per lane covers all 4 steps;
//   i/j-contiguous operand: one float4 along i/j per lane and step covers 4
//                           MFMA blocks whose rows (cols) interleave with
//                           stride 4 (block u of a 64-wide group holds rows
//                           4*lane16 + u).
//
// Epilogues: STORE  C = res + act(acc + bias)
//            ACCUM  C += acc                      (gradient accumulation)
//            PARTIAL ws[split] = acc              (deterministic split-K;
//                                                  reduced by splitk_reduce)
#include "ncm_dev.h"

enum { EPI_STORE = 0, EPI_ACCUM = 1, EPI_PARTIAL = 2 };

struct GemmArgs {
    const float *A;
    const float *B;
    float *C;
    const float *bias;   // [No] or null (STORE only)
    const float *res;    // [Mo, ldc] or null (STORE only)
    float *ws;           // split-K partials [splits][Mo][No] (PARTIAL only)
    int Mo, No, K;
    int lda, ldb, ldc;
    int k_per_split;     // multiple of BK
    int act;
    int tiles_m, tiles_n;
};

// Maps the launch index to an output tile.  Workgroups are dispatched
// round-robin over the 8 XCDs (each with its own L2); the remap gives each
// XCD a contiguous range of logical tiles, and the grouped raster inside that
// range keeps GROUP_M tile rows sharing B panels close in time.
template <int GROUP_M>
__device__ __forceinline__ void tile_coords(int tiles_m, int tiles_n, int &tm, int &tn) {
    int nb = tiles_m * tiles_n;
    int lin = blockIdx.x;
    if ((nb & 7) == 0) lin = (lin & 7) * (nb >> 3) + (lin >> 3);
    int group = GROUP_M * tiles_n;
    int g = lin / group;
    int first = g * GROUP_M;
    int gm = min(tiles_m - first, GROUP_M);
    int in = lin - g * group;
    tm = first + in % gm;
    tn = in / gm;
}

template <int BM, int BN, int BK, int WM, int WN, bool AKC, bool BKC, int EPI, bool VEC>
__device__ __forceinline__ void gemm_body(const GemmArgs &p) {
    constexpr int WAVES_N = BN / WN;
    constexpr int NT = (BM / WM) * WAVES_N * 64;
    constexpr int TM = WM / 16, TN = WN / 16;
    static_assert(BK % 16 == 0, "BK must be a multiple of 16");
    static_assert(AKC || WM % 64 == 0, "i-contiguous A needs 64-row wave tiles");
    static_assert(BKC || WN % 64 == 0, "j-contiguous B needs 64-col wave tiles");

    constexpr int A_ROWS = AKC ? BM : BK, A_COLS = AKC ? BK : BM;
    constexpr int B_ROWS = BKC ? BN : BK, B_COLS = BKC ? BK : BN;
    constexpr int A_LD = A_COLS + 4, B_LD = B_COLS + 4;
    constexpr int A_SZ = A_ROWS * A_LD, B_SZ = B_ROWS * B_LD;
    __shared__ __attribute__((aligned(16))) float smem[2 * (A_SZ + B_SZ)];
    float *const sA = smem;               // buffers sA + {0, A_SZ}
    float *const sB = smem + 2 * A_SZ;    // buffers sB + {0, B_SZ}

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int wm = wave / WAVES_N, wn = wave % WAVES_N;
    const int li = lane & 15, lg = lane >> 4;

    int tm, tn;
    tile_coords<8>(p.tiles_m, p.tiles_n, tm, tn);
    const int i0 = tm * BM, j0 = tn * BN;
    const int split = blockIdx.z;
    const int kbeg = split * p.k_per_split;
    const int kend = min(p.K, kbeg + p.k_per_split);
    const int nk = (kend - kbeg + BK - 1) / BK;

    TileLoader<A_ROWS, A_COLS, NT, VEC> la;
    TileLoader<B_ROWS, B_COLS, NT, VEC> lb;

    f4 acc[TM][TN];
#pragma unroll
    for (int a = 0; a < TM; ++a)
#pragma unroll
        for (int b = 0; b < TN; ++b) acc[a][b] = f4{0.f, 0.f, 0.f, 0.f};

    auto gload = [&](int kb) {
        if (AKC) la.load(p.A, p.lda, i0, kb, p.Mo, kend, tid);
        else     la.load(p.A, p.lda, kb, i0, kend, p.Mo, tid);
        if (BKC) lb.load(p.B, p.ldb, j0, kb, p.No, kend, tid);
        else     lb.load(p.B, p.ldb, kb, j0, kend, p.No, tid);
    };

    if (nk > 0) {
        gload(kbeg);
        la.store(sA, tid);
        lb.store(sB, tid);
    }
    __syncthreads();

    for (int kt = 0; kt < nk; ++kt) {
        const int cur = kt & 1;
        const bool more = kt + 1 < nk;
        if (more) gload(kbeg + (kt + 1) * BK);

        const float *a_s = sA + cur * A_SZ;
        const float *b_s = sB + cur * B_SZ;
#pragma unroll
        for (int kc = 0; kc < BK / 16; ++kc) {
            f4 ak[AKC ? TM : 1], bk[BKC ? TN : 1];
            if (AKC) {
#pragma unroll
                for (int t = 0; t < TM; ++t)
                    ak[t] = *(const f4 *)(a_s + (wm * WM + t * 16 + li) * A_LD + kc * 16 + 4 * lg);
            }
            if (BKC) {
#pragma unroll
                for (int t = 0; t < TN; ++t)
                    bk[t] = *(const f4 *)(b_s + (wn * WN + t * 16 + li) * B_LD + kc * 16 + 4 * lg);
            }
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                f4 as[AKC ? 1 : TM / 4], bs[BKC ? 1 : TN / 4];
                if (!AKC) {
#pragma unroll
                    for (int q = 0; q < TM / 4; ++q)
                        as[q] = *(const f4 *)(a_s + (kc * 16 + 4 * lg + s) * A_LD + wm * WM + q * 64 + 4 * li);
                }
                if (!BKC) {
#pragma unroll
                    for (int q = 0; q < TN / 4; ++q)
                        bs[q] = *(const f4 *)(b_s + (kc * 16 + 4 * lg + s) * B_LD + wn * WN + q * 64 + 4 * li);
                }
#pragma unroll
                for (int a = 0; a < TM; ++a) {
                    float av = AKC ? ak[a][s] : as[a >> 2][a & 3];
#pragma unroll
                    for (int b = 0; b < TN; ++b) {
                        float bv = BKC ? bk[b][s] : bs[b >> 2][b & 3];
                        acc[a][b] = mfma4(av, bv, acc[a][b]);
                    }
                }
            }
        }

        if (more) {
            la.store(sA + (cur ^ 1) * A_SZ, tid);
            lb.store(sB + (cur ^ 1) * B_SZ, tid);
        }
        __syncthreads();
    }

    // ---- epilogue ----
    // acc[a][b][r] holds MFMA row rho = 4*lg + r, column gamma = li.
    float *outp;
    int ldo;
    if (EPI == EPI_PARTIAL) {
        outp = p.ws + (int64_t)split * p.Mo * p.No;
        ldo = p.No;
    } else {
        outp = p.C;
        ldo = p.ldc;
    }
#pragma unroll
    for (int a = 0; a < TM; ++a) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int rho = 4 * lg + r;
            const int row = i0 + wm * WM + (AKC ? a * 16 + rho : (a >> 2) * 64 + 4 * rho + (a & 3));
            if (row >= p.Mo) continue;
            float *orow = outp + (int64_t)row * ldo;
            const float *rrow = (EPI == EPI_STORE && p.res) ? p.res + (int64_t)row * p.ldc : nullptr;
#pragma unroll
            for (int b = 0; b < TN; ++b) {
                const int col = j0 + wn * WN + (BKC ? b * 16 + li : (b >> 2) * 64 + 4 * li + (b & 3));
                if (col >= p.No) continue;
                float v = acc[a][b][r];
                if (EPI == EPI_STORE) {
                    if (p.bias) v += p.bias[col];
                    v = ncm_act(v, p.act);
                    if (rrow) v = rrow[col] + v;
                    orow[col] = v;
                } else if (EPI == EPI_ACCUM) {
                    orow[col] += v;
                } else {
                    orow[col] = v;
                }
            }
        }
    }
}

// Sums the split-K partials in split order (deterministic) and applies the
// final epilogue.  One thread per output element.
extern "C" __global__ void __launch_bounds__(256)
splitk_reduce(const float *__restrict__ ws, int splits, int Mo, int No, float *C, int ldc,
              const float *bias, const float *res, int act, int accum) {
    int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
    int64_t total = (int64_t)Mo * No;
    if (idx >= total) return;
    int row = (int)(idx / No), col = (int)(idx % No);
    float s = 0.f;
    for (int z = 0; z < splits; ++z) s += ws[(int64_t)z * total + idx];
    float *o = C + (int64_t)row * ldc + col;
    if (accum) {
        *o += s;
    } else {
        if (bias) s += bias[col];
        s = ncm_act(s, act);
        if (res) s = res[(int64_t)row * ldc + col] + s;
        *o = s;
    }
}

// db[m] += (float) sum_r dy[r,m], the bias gradient of train_tape.c:708-713
// (fp64 accumulation as there).  Stage 1: partial fp64 column sums over
// row chunks; stage 2: ordered sum of the partials.
extern "C" __global__ void __launch_bounds__(256)
colsum_partial(const float *__restrict__ dy, int64_t rows, int N, int rows_per_chunk,
               double *__restrict__ part) {
    int col = blockIdx.x * 256 + threadIdx.x;
    int chunk = blockIdx.y;
    if (col >= N) return;
    int64_t r0 = (int64_t)chunk * rows_per_chunk;
    int64_t r1 = min(rows, r0 + rows_per_chunk);
    double s = 0.0;
    for (int64_t r = r0; r < r1; ++r) s += (double)dy[r * N + col];
    part[(int64_t)chunk * N + col] = s;
}

extern "C" __global__ void __launch_bounds__(256)
colsum_final(const double *__restrict__ part, int chunks, int N, float *db) {
    int col = blockIdx.x * 256 + threadIdx.x;
    if (col >= N) return;
    double s = 0.0;
    for (int c = 0; c < chunks; ++c) s += part[(int64_t)c * N + col];
    db[col] += (float)s;
}

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
#define GEMM_KERNEL(name, BM, BN, BK, WM, WN, AKC, BKC, EPI, VEC)                        \
    extern "C" __global__ void __launch_bounds__((BM / WM) * (BN / WN) * 64, 2)          \
    name(GemmArgs p) { gemm_body<BM, BN, BK, WM, WN, AKC, BKC, EPI, VEC>(p); }

// 128x128 tiles, 4 waves of 64x64, BK=16
GEMM_KERNEL(gemm_fwd_store_v,   128, 128, 16, 64, 64, true,  true,  EPI_STORE,   true)
GEMM_KERNEL(gemm_fwd_part_v,    128, 128, 16, 64, 64, true,  true,  EPI_PARTIAL, true)
GEMM_KERNEL(gemm_fwd_store_s,   128, 128, 16, 64, 64, true,  true,  EPI_STORE,   false)
GEMM_KERNEL(gemm_fwd_part_s,    128, 128, 16, 64, 64, true,  true,  EPI_PARTIAL, false)
GEMM_KERNEL(gemm_dx_accum_v,    128, 128, 16, 64, 64, true,  false, EPI_ACCUM,   true)
GEMM_KERNEL(gemm_dx_part_v,     128, 128, 16, 64, 64, true,  false, EPI_PARTIAL, true)
GEMM_KERNEL(gemm_dx_accum_s,    128, 128, 16, 64, 64, true,  false, EPI_ACCUM,   false)
GEMM_KERNEL(gemm_dx_part_s,     128, 128, 16, 64, 64, true,  false, EPI_PARTIAL, false)
GEMM_KERNEL(gemm_dw_accum_v,    128, 128, 16, 64, 64, false, false, EPI_ACCUM,   true)
GEMM_KERNEL(gemm_dw_part_v,     128, 128, 16, 64, 64, false, false, EPI_PARTIAL, true)
GEMM_KERNEL(gemm_dw_accum_s,    128, 128, 16, 64, 64, false, false, EPI_ACCUM,   false)
GEMM_KERNEL(gemm_dw_part_s,     128, 128, 16, 64, 64, false, false, EPI_PARTIAL, false)

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
