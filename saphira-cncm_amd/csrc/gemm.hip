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
// BK = 32 k are consumed as two 16-wide chunks from two LDS stages, one
// barrier per slab.  The vectorised kernels (_v, the common case) load slabs
// straight into LDS (buffer_load_dwordx4 ... lds) and keep each slab in its
// memory layout; the scalar kernels (_s: an operand row not 16-byte aligned)
// stage through registers and transpose i/j-contiguous slabs into k-contiguous
// LDS rows.  Both layouts are free of LDS bank conflicts (see below).  Global
// loads are raw buffer loads: lanes outside the matrix get an offset beyond
// the buffer and read zero, so the loop body has no branches.
//
// Pipeline (per slab): fragment reads run one chunk ahead of the MFMAs that
// use them (across the barrier too), and the global loads of the slab after
// next are issued right after the barrier, ahead of the second chunk's MFMAs.
//
// k-permutation: inside every 16-wide chunk, MFMA step s (0..3) gives lane
// group g = lane/16 the reduction index k = 4g + s, for both operands.  The
// MFMA sums over all 16 (g, s) pairs, so the product is unchanged, but every
// operand fragment becomes one 128-bit LDS read (a float4 along k covers the
// 4 steps).
//
// Scheduling: tiles [0, dp_tiles) run whole, one workgroup each; every other
// tile is cut into `segs` k-segments that fill the last round of the chip.
// Segments store partial tiles; gemm_64x64_fixup_* (a second launch, one
// workgroup per MFMA block of a split tile) sums them in segment order --
// deterministic -- and applies the epilogue.
//
// Accuracy: MFMAs accumulate 128 k into `acc`, which is then added into `tot`;
// a single fp32 chain over K terms has an error growing like K u, the two
// levels keep it near (128 + K/128) u.
//
// Epilogues: STORE  C = res + act(acc + bias) (or act(acc + bias) * res, the
// gated-unit product);  ACCUM  C += acc;  GATED  C = act(x B^T + bias) *
// (x B2^T + bias2), both products in one tile (gemm_64x64_gated_v);
// ACT_BWD  C += act'(bwd_x) (0.0f + acc): the dX product written as a fresh
// gradient and passed back through the activation that produced the layer's
// input, without storing it (gemm_64x64_dxa_v).
#include "mfma_slab.h"

enum { EPI_STORE = 0, EPI_ACCUM = 1, EPI_GATED = 2, EPI_ACT_BWD = 3 };
// Per-tile output selection: SEL_F3 (gemm_64x64_fwd3_v, f3_select) and
// SEL_HEADS (gemm_64x64_fwdh_v, gemm_64x64_dxh_v: heads_select).
enum { SEL_NONE = 0, SEL_F3 = 1, SEL_HEADS = 2 };

struct GemmArgs {
    const float *A;
    const float *B;
    float *C;
    const float *bias;   // [No] or null (STORE only)
    const float *res;    // [Mo, ldc] or null (STORE only): added, or multiplied when res_mul
    float *ws;           // partial tiles of split tiles [units][64*64]
    int Mo, No, K;
    int lda, ldb, ldc;
    int act;
    int res_mul;         // STORE: C = act(acc + bias) * res instead of res + act(acc + bias)
    int tiles_m, tiles_n;
    int iters;           // BK slabs per tile (a multiple of 4)
    int dp_tiles;        // blocks [0, dp_tiles): one whole tile each
    int segs;            // later blocks: k-segment (u % segs) of tile dp_tiles + u / segs
    unsigned a_bytes, b_bytes;  // extents of A and B for the buffer descriptors
    const float *B2;     // GATED: the up-projection weight (B is the gate's)
    const float *bias2;  // GATED: its bias or null
    int beta;            // ACCUM: 1 C += acc; 0 C = 0.0f + acc, the first write of a gradient (the bits of an
                         // accumulation into zeros, without reading C or clearing it first)
    float *db;           // dW (vectorised kernel) or null: db[i] += 0.0f + (float)(fp64 sum over k of A(i,k)),
                         // the bias gradient, from the A slabs of the tiles in tile column 0
    double *dbpart;      // its per-segment fp64 partials of split tiles [units][64]
    float *pre;          // STORE or null: also stores acc + bias (before the activation) at the same index
    const float *bwd_x;  // ACT_BWD: the activation's input, indexed like C
    int bwd_kind;        // ACT_BWD: 0 GELU (erf), 1 SiLU, 2 GELU (tanh form)
    // F3 kernels (gemm_64x64_fwd3_v): up to three products of the same A side by
    // side, product g owning n3[g] output columns (a multiple of 64 but the
    // last) with its own B (extent b3_bytes[g]), bias and output [Mo][n3[g]]
    const float *B3[3];
    const float *bias3[3];
    float *C3[3];
    int n3[3];
    unsigned b3_bytes[3];
    // SEL_HEADS (gemm_64x64_fwdh_v): output row i = b T + t of a [q | k | v]
    // product (part widths n3[], heads of 64 columns) goes to C3[part] as
    // [B][n3[part] / 64][T][64]; hm_T = T, a multiple of 64
    int hm_T;
};

// SEL_HEADS: the tile at (i0, j0) lies in one head of one part and, T being a
// multiple of 64, in one sequence b; in the head-major layout its 64 rows are
// one contiguous [64][64] block.  So the tile is stored as a plain row-major
// tile through q.C, offset so that C + i * 64 + j (ldc 64) lands in that
// block for every (i, j) of the tile.
__device__ __forceinline__ void heads_select(const GemmArgs &src, GemmArgs &q, int i0, int j0) {
    const int n0 = src.n3[0], n01 = n0 + src.n3[1];
    const int g = j0 < n0 ? 0 : j0 < n01 ? 1 : 2;
    const int jl = j0 - (g == 0 ? 0 : g == 1 ? n0 : n01);
    const int hw = (g == 0 ? n0 : g == 1 ? src.n3[1] : src.n3[2]) >> 6;
    float *const base = g == 0 ? src.C3[0] : g == 1 ? src.C3[1] : src.C3[2];
    const int b = i0 / src.hm_T, t0 = i0 - b * src.hm_T;
    float *const blk = base + (((int64_t)b * hw + (jl >> 6)) * src.hm_T + t0) * 64;
    q.C = blk - (int64_t)i0 * 64 - j0;
    q.ldc = 64;
}

// F3: the product that output column jt (a tile's first) belongs to, written
// into q (a copy of the arguments) as a plain GEMM's B, bias, output and
// width; returns the product's first column.  The tables are read from the
// kernel's own arguments: selecting from the copy's arrays would index them
// at run time and keep the copy in scratch memory.
__device__ __forceinline__ int f3_select(const GemmArgs &src, GemmArgs &q, int jt) {
    const int n0 = src.n3[0], n01 = n0 + src.n3[1];
    const int g = jt < n0 ? 0 : jt < n01 ? 1 : 2;
    q.B = g == 0 ? src.B3[0] : g == 1 ? src.B3[1] : src.B3[2];
    q.bias = g == 0 ? src.bias3[0] : g == 1 ? src.bias3[1] : src.bias3[2];
    q.C = g == 0 ? src.C3[0] : g == 1 ? src.C3[1] : src.C3[2];
    q.No = g == 0 ? n0 : g == 1 ? src.n3[1] : src.n3[2];
    q.ldc = q.No;
    q.b_bytes = g == 0 ? src.b3_bytes[0] : g == 1 ? src.b3_bytes[1] : src.b3_bytes[2];
    return g == 0 ? 0 : g == 1 ? n0 : n01;
}

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

// The same sum in one launch for rows <= COLSUM_SMALL_ROWS: a workgroup of 16
// waves owns 64 columns (one per lane, so any N and alignment), wave w sums
// rows w, w + 16, ... in fp64 with all of its loads in flight, and wave 0
// adds the 16 partials in wave order.  Two launches of ~4 us each were the
// whole cost of a small-batch bias gradient.
#define COLSUM_SMALL_ROWS 512
extern "C" __global__ void __launch_bounds__(1024)
colsum_small(const float *__restrict__ dy, int rows, int N, float *db) {
    __shared__ double red[16][64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int col = blockIdx.x * 64 + lane;
    double s = 0.0;
    if (col < N) {
        // unconditional loads of a clamped row (a guarded load would be a
        // branch with a wait after it), rows past the end then count zero
        float v[COLSUM_SMALL_ROWS / 16];
        const float *p = dy + col;
#pragma unroll
        for (int j = 0; j < COLSUM_SMALL_ROWS / 16; ++j)
            v[j] = p[(int64_t)min(wave + 16 * j, rows - 1) * N];
#pragma unroll
        for (int j = 0; j < COLSUM_SMALL_ROWS / 16; ++j)
            if (wave + 16 * j < rows) s += (double)v[j];
    }
    red[wave][lane] = s;
    __syncthreads();
    if (wave == 0 && col < N) {
        double t = red[0][lane];
#pragma unroll
        for (int w = 1; w < 16; ++w) t += red[w][lane];
        db[col] += 0.0f + (float)t;   // the reference adds a zeroed temporary (train_tape.c:708-720)
    }
}

extern "C" __global__ void __launch_bounds__(256)
colsum_final(const double *__restrict__ part, int chunks, int N, float *db) {
    int col = blockIdx.x * 256 + threadIdx.x;
    if (col >= N) return;
    double s = 0.0;
#pragma unroll 16
    for (int c = 0; c < chunks; ++c) s += part[(int64_t)c * N + col];
    db[col] += 0.0f + (float)s;
}

// Stage 2 over many chunks: a workgroup of 16 waves per 64 columns, wave v
// adds chunks v, v + 16, ... in order with 16 loads in flight per pass, then
// wave 0 adds the 16 wave sums in wave order (colsum_final walks every chunk
// of a column in one thread, one round trip per 16 chunks).
extern "C" __global__ void __launch_bounds__(1024)
colsum_final_w(const double *__restrict__ part, int chunks, int N, float *db) {
    __shared__ double red[16][64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int col = blockIdx.x * 64 + lane;
    double s = 0.0;
    if (col < N) {
        for (int k0 = wave; k0 < chunks; k0 += 256) {
            double v[16];
#pragma unroll
            for (int u = 0; u < 16; ++u) v[u] = part[(int64_t)min(k0 + 16 * u, chunks - 1) * N + col];
#pragma unroll
            for (int u = 0; u < 16; ++u)
                if (k0 + 16 * u < chunks) s += v[u];
        }
    }
    red[wave][lane] = s;
    __syncthreads();
    if (wave == 0 && col < N) {
        double t = red[0][lane];
#pragma unroll
        for (int w = 1; w < 16; ++w) t += red[w][lane];
        db[col] += 0.0f + (float)t;   // the reference adds a zeroed temporary (train_tape.c:708-720)
    }
}

// ---- small-batch backward (batch <= 8 rows of dy) ----
// dW[n,k] += sum_r dy[r,n] x[r,k]: the reference's per-output fp64 sum over
// r ascending, rounded to float and added through a zeroed temporary
// (train_tape.c:714-720), so this path is bit-exact with the host backward.
// One thread per 4 consecutive k of one row n; HBM-bound on dW.  With db,
// the thread of k = 0 also adds the bias gradient db[n] += (float) sum_r
// dy[r,n] (fp64, r ascending: colsum_small's sum over these rows) from the
// dy values it loads anyway, so the call needs no second launch.
template <bool VEC>
__device__ __forceinline__ void dw_rank_body(const float *__restrict__ dy, const float *__restrict__ x,
                                             float *dW, float *db, int nb, int N, int K) {
#pragma clang fp contract(off)
    const int64_t f = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int K4 = (K + 3) / 4;
    if (f >= (int64_t)N * K4) return;
    const int n = (int)(f / K4), k = (int)(f % K4) * 4;
    double s[4] = {0.0, 0.0, 0.0, 0.0}, t = 0.0;
    for (int r = 0; r < nb; ++r) {
        const double g = dy[(int64_t)r * N + n];
        t += g;
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
    if (db != nullptr && k == 0) db[n] += 0.0f + (float)t;
}

extern "C" __global__ void __launch_bounds__(256)
dw_rank_v(const float *dy, const float *x, float *dW, float *db, int nb, int N, int K) {
    dw_rank_body<true>(dy, x, dW, db, nb, N, K);
}
extern "C" __global__ void __launch_bounds__(256)
dw_rank_s(const float *dy, const float *x, float *dW, float *db, int nb, int N, int K) {
    dw_rank_body<false>(dy, x, dW, db, nb, N, K);
}

// dx[r,k] += sum_n dy[r,n] W[n,k] for r < nb: a transposed GEMV streaming W
// once.  Block = 4 waves x 256 columns (float4 per lane); the waves take
// interleaved rows n of a chunk of DXT_ROWS rows, LDS combines them, and the
// chunk partials [chunk][nb][K] are summed by dxt_final (four interleaved
// wave sums over the chunks, added in wave order).
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

// dx[f] += sum over the chunk partials: a workgroup per 64 outputs, wave w
// summing chunks w, w + 4, ... (16 loads in flight per pass), the four wave
// sums added in wave order -- a quarter of the dependent round trips of one
// thread walking every chunk (up to 152 for a 4864-row W).
extern "C" __global__ void __launch_bounds__(256)
dxt_final(const float *__restrict__ part, int chunks, int nb, int K, float *__restrict__ dx) {
    __shared__ float red[4][64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int64_t n = (int64_t)nb * K, f = (int64_t)blockIdx.x * 64 + lane;
    const int64_t fc = f < n ? f : n - 1;
    float s = 0.f;
    for (int c0 = wave; c0 < chunks; c0 += 64) {
        float v[16];
#pragma unroll
        for (int u = 0; u < 16; ++u) v[u] = part[(int64_t)min(c0 + 4 * u, chunks - 1) * n + fc];
#pragma unroll
        for (int u = 0; u < 16; ++u)
            if (c0 + 4 * u < chunks) s += v[u];
    }
    red[wave][lane] = s;
    __syncthreads();
    if (wave == 0 && f < n) dx[f] += ((red[0][lane] + red[1][lane]) + red[2][lane]) + red[3][lane];
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

// ---------------------------------------------------------------- GEMM, register-staged loads
// (the _s kernels.)  Tiles of BM x BN, four waves in 2 x 2, a wave owning a
// (BM/2) x (BN/2) sub-tile of TM x TN MFMA blocks.
//
// LDS layout of a slab (rows = tile rows, BK = 32 floats of k per row): pitch
// G_LD = 40 floats, and the float4 group of k XORed with h(row) =
// ((row >> 2) ^ (row >> 5)) & 7.  gfx950 serves a ds_read_b128 16 lanes per
// cycle in the groups {0-3, 12-15, 20-23, 24-27} and {4-7, 8-11, 16-19,
// 28-31} (and the same +32), a ds_write_b128 8 consecutive lanes per cycle and
// a ds_write_b32 32 consecutive lanes per cycle, over 64 four-byte banks.
// With this layout each of the three accesses of the kernel -- fragment reads
// (16 consecutive rows, one float4 of k each), k-contiguous slab stores (8
// lanes = one row) and the transposing b32 stores of i/j-contiguous slabs
// (32 lanes = 16 rows x 2 k) -- touches every bank at most once per cycle.
#define G_LD (GEMM_BK + 8)
__device__ __forceinline__ int gswz(int row, int k) {
    return ((((k >> 2) ^ (row >> 2) ^ (row >> 5)) & 7) << 2) | (k & 3);
}

template <int ROWS, bool KC, bool VEC>
struct GSlab {
    // KC: memory [ROWS rows][K] (k along columns): thread t loads row (t >> 3) + 32 j, k (t & 7) * 4.
    // else memory [K][ROWS cols]: thread t loads k-row t / (ROWS/4) + KSTEP j, cols (t % (ROWS/4)) * 4.
    static constexpr int PER = ROWS / 32;               // float4 per thread per slab (both layouts)
    static constexpr int C4 = ROWS / 4, KSTEP = GEMM_NT / C4;
    int a0, b0;
    int ld, fix0, fix_lim;
    // VEC: byte offset of the thread's float4 j at k = 0, or OOB_OFFSET when it
    // lies outside the tile's valid rows (KC) / columns (!KC), and the bound
    // on a slab's first k below which float4 j lies inside the k range.  A
    // load is then an add, a compare and a select, with no branch, so that
    // the loads can be spread between the MFMAs.
    unsigned base[PER];
    int klim[PER];
    __device__ __forceinline__ void init(int tid, int ld_, int fix0_, int fix_lim_, int k_lim) {
        ld = ld_;
        fix0 = fix0_;
        fix_lim = fix_lim_;
        if (KC) { a0 = tid >> 3; b0 = (tid & 7) * 4; }
        else { a0 = tid / C4; b0 = (tid % C4) * 4; }
        if (VEC) {
#pragma unroll
            for (int j = 0; j < PER; ++j) {
                if (KC) {
                    const int row = fix0 + a0 + 32 * j;
                    base[j] = row < fix_lim ? (unsigned)(row * ld + b0) * 4u : OOB_OFFSET;
                    klim[j] = k_lim - b0;   // K % 4 == 0: the float4 is whole or out
                } else {
                    const int col = fix0 + b0;   // fix_lim % 4 == 0: the float4 is whole or out
                    base[j] = col < fix_lim ? (unsigned)((a0 + KSTEP * j) * ld + col) * 4u : OOB_OFFSET;
                    klim[j] = k_lim - a0 - KSTEP * j;
                }
            }
        }
    }
    // k0: first k of the slab; k_lim: end of the k range (the one init got)
    __device__ __forceinline__ void load(__amdgpu_buffer_rsrc_t rs, int k0, int k_lim, f4 (&r)[PER]) const {
        if (VEC) {
            const unsigned dk = KC ? (unsigned)k0 * 4u : (unsigned)k0 * (unsigned)ld * 4u;
#pragma unroll
            for (int j = 0; j < PER; ++j)
                r[j] = __builtin_bit_cast(
                    f4, __builtin_amdgcn_raw_buffer_load_b128(rs, k0 < klim[j] ? base[j] + dk : OOB_OFFSET, 0, 0));
            return;
        }
#pragma unroll
        for (int j = 0; j < PER; ++j) {
            const int rw = KC ? fix0 + a0 + 32 * j : k0 + a0 + KSTEP * j;
            const int cl = KC ? k0 + b0 : fix0 + b0;
            const bool in_r = KC ? rw < fix_lim : rw < k_lim;
            const int lim_c = KC ? k_lim : fix_lim;
            const unsigned o = (unsigned)(rw * ld + cl) * 4u;
#pragma unroll
            for (int u = 0; u < 4; ++u)
                r[j][u] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                                        rs, (in_r && cl + u < lim_c) ? o + 4u * u : OOB_OFFSET, 0, 0));
        }
    }
    __device__ __forceinline__ void store(float *buf, const f4 (&r)[PER]) const {
#pragma unroll
        for (int j = 0; j < PER; ++j) {
            if (KC) {
                const int row = a0 + 32 * j;
                *(f4 *)(buf + row * G_LD + gswz(row, b0)) = r[j];
            } else {
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    const int row = b0 + u;
                    buf[row * G_LD + gswz(row, a0 + KSTEP * j)] = r[j][u];
                }
            }
        }
    }
};

// The epilogue of N output elements (ii[n], jj[n], v[n]) of one thread, in two
// phases: every operand the elements need -- the old C of an accumulation,
// the bias, the residual -- is loaded first, unconditionally, from clamped
// coordinates (an absent bias reads C[0] in its place, an absent residual
// the bias address, so neither costs a stream); then the in-bounds elements
// are computed and stored: C += v (ACCUM), or C = res + act(v + bias) /
// act(v + bias) * res (STORE).  One guarded element at a time made each
// element a memory round trip (load, wait, store).
template <int N, int ACT, int EPI>
__device__ __forceinline__ void g_out_n(const GemmArgs &p, const int (&ii)[N], const int (&jj)[N],
                                        const float (&v)[N]) {
#pragma clang fp contract(off)
    const bool hb = p.bias != nullptr, hr = p.res != nullptr;
    float o1[N], o2[N];
#pragma unroll
    for (int n = 0; n < N; ++n) {
        const int i = min(ii[n], p.Mo - 1), j = min(jj[n], p.No - 1);
        const int64_t e = (int64_t)i * p.ldc + j;
        if (EPI == EPI_ACCUM || EPI == EPI_ACT_BWD) {
            o1[n] = p.beta ? p.C[e] : 0.0f;
            if (EPI == EPI_ACT_BWD) o2[n] = p.bwd_x[e];
        } else {
            const float *bq = hb ? p.bias + j : p.A;   // an absent bias reads a valid stand-in
            o1[n] = *bq;
            o2[n] = *(hr ? p.res + e : bq);
        }
    }
#pragma unroll
    for (int n = 0; n < N; ++n) {
        if (ii[n] >= p.Mo || jj[n] >= p.No) continue;
        float *c = p.C + (int64_t)ii[n] * p.ldc + jj[n];
        float x = v[n];
        if (EPI == EPI_ACCUM) {
            *c = o1[n] + x;
        } else if (EPI == EPI_ACT_BWD) {
            *c = o1[n] + act_bwd_one(o2[n], 0.0f + x, p.bwd_kind);
        } else {
            if (hb) x += o1[n];
            if (p.pre) p.pre[(int64_t)ii[n] * p.ldc + jj[n]] = x;
            x = ncm_act(x, ACT);
            if (hr) x = p.res_mul ? x * o2[n] : o2[n] + x;
            *c = x;
        }
    }
}

// tot[a][b][r] holds MFMA output row 4*lg + r, column li of block (a, b).
// Blocks of 16 consecutive rows / columns: row wm*(BM/2) + a*16 + 4*lg + r,
// column wn*(BN/2) + b*16 + li.  Interleaved (IA / IB, the operand read from
// an i/j-contiguous LDS slab, one read feeding every block of the wave):
// block a takes the rows wm*(BM/2) + (BM/32)*i + a, block b the columns
// wn*(BN/2) + (BN/32)*j + b.
template <int BM, int BN, int EPI, int ACT, bool IA, bool IB>
__device__ __forceinline__ void g_epilogue_act(const GemmArgs &p, const f4 (&tot)[BM / 32][BN / 32], int i0, int j0,
                                               int tid) {
    const int lane = tid & 63, wave = tid >> 6, wm = wave >> 1, wn = wave & 1;
    const int li = lane & 15, lg = lane >> 4;
    constexpr int N = (BM / 32) * (BN / 32) * 4;
    int ii[N], jj[N];
    float v[N];
#pragma unroll
    for (int a = 0; a < BM / 32; ++a)
#pragma unroll
        for (int b = 0; b < BN / 32; ++b)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int n = (a * (BN / 32) + b) * 4 + r;
                const int row = IA ? wm * (BM / 2) + (BM / 32) * (4 * lg + r) + a : wm * (BM / 2) + a * 16 + 4 * lg + r;
                const int col = IB ? wn * (BN / 2) + (BN / 32) * li + b : wn * (BN / 2) + b * 16 + li;
                ii[n] = i0 + row;
                jj[n] = j0 + col;
                v[n] = tot[a][b][r];
            }
    g_out_n<N, ACT, EPI>(p, ii, jj, v);
}

template <int BM, int BN, int EPI, bool IA = false, bool IB = false>
__device__ __forceinline__ void g_epilogue(const GemmArgs &p, const f4 (&tot)[BM / 32][BN / 32], int i0, int j0,
                                           int tid) {
    if (EPI == EPI_ACCUM || EPI == EPI_ACT_BWD) {
        g_epilogue_act<BM, BN, EPI, ACT_NONE, IA, IB>(p, tot, i0, j0, tid);
        return;
    }
    switch (p.act) {
    case ACT_SILU: g_epilogue_act<BM, BN, EPI, ACT_SILU, IA, IB>(p, tot, i0, j0, tid); break;
    case ACT_GELU: g_epilogue_act<BM, BN, EPI, ACT_GELU, IA, IB>(p, tot, i0, j0, tid); break;
    case ACT_GELU_TANH: g_epilogue_act<BM, BN, EPI, ACT_GELU_TANH, IA, IB>(p, tot, i0, j0, tid); break;
    case ACT_RELU2: g_epilogue_act<BM, BN, EPI, ACT_RELU2, IA, IB>(p, tot, i0, j0, tid); break;
    default: g_epilogue_act<BM, BN, EPI, ACT_NONE, IA, IB>(p, tot, i0, j0, tid); break;
    }
}

template <int BM, int BN, bool AKC, bool BKC, int EPI, bool VEC>
__device__ __forceinline__ void gemm_tile_body(const GemmArgs &p) {
    constexpr int TM = BM / 32, TN = BN / 32;
    __shared__ __attribute__((aligned(16))) float sA[2 * BM * G_LD];
    __shared__ __attribute__((aligned(16))) float sB[2 * BN * G_LD];
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
    const int i0 = tm * BM, j0 = tn * BN;
    const int kend = min(p.K, it1 * GEMM_BK);
    const __amdgpu_buffer_rsrc_t ra = make_rsrc(p.A, p.a_bytes), rb = make_rsrc(p.B, p.b_bytes);
    GSlab<BM, AKC, VEC> la;
    GSlab<BN, BKC, VEC> lb;
    la.init(tid, p.lda, i0, p.Mo, kend);
    lb.init(tid, p.ldb, j0, p.No, kend);

    f4 acc[TM][TN], tot[TM][TN];
#pragma unroll
    for (int a = 0; a < TM; ++a)
#pragma unroll
        for (int b = 0; b < TN; ++b) acc[a][b] = tot[a][b] = f4{0.f, 0.f, 0.f, 0.f};

    // fragments of one 16-wide chunk: fa[t] = A rows wm*(BM/2) + 16 t + li,
    // fb[t] = B rows wn*(BN/2) + 16 t + li, k = 16 kc + 4 lg .. + 3
    auto read_frags = [&](const float *a_s, const float *b_s, int kc, f4 (&fa)[TM], f4 (&fb)[TN]) {
#pragma unroll
        for (int t = 0; t < TM; ++t) {
            const int r = wm * (BM / 2) + t * 16 + li;
            fa[t] = *(const f4 *)(a_s + r * G_LD + gswz(r, kc * 16 + 4 * lg));
        }
#pragma unroll
        for (int t = 0; t < TN; ++t) {
            const int r = wn * (BN / 2) + t * 16 + li;
            fb[t] = *(const f4 *)(b_s + r * G_LD + gswz(r, kc * 16 + 4 * lg));
        }
    };
    auto mfmas = [&](const f4 (&fa)[TM], const f4 (&fb)[TN]) {
#pragma unroll
        for (int s = 0; s < 4; ++s)
#pragma unroll
            for (int a = 0; a < TM; ++a)
#pragma unroll
                for (int b = 0; b < TN; ++b) acc[a][b] = mfma4(fa[a][s], fb[b][s], acc[a][b]);
    };

    // Software pipeline, per slab (buffer cur holds it, registers ga / gb
    // the next one):
    //   issue the LDS reads of chunk 1 (f1), then the MFMAs of chunk 0 (f0);
    //   store the next slab into the other buffer; barrier;
    //   issue the LDS reads of the next slab's chunk 0 (f0), then the MFMAs
    //   of chunk 1 with the global loads of the slab after next spread
    //   between them (one load per TM*TN MFMAs: issued in a burst, the loads
    //   stall the wave on the vector-memory pipe).
    // Every LDS read is covered by one chunk of MFMAs of the same wave and
    // every global load by one slab of them.
    constexpr int NLOAD = GSlab<BM, AKC, VEC>::PER + GSlab<BN, BKC, VEC>::PER;
    f4 f0a[TM], f0b[TN], f1a[TM], f1b[TN];
    f4 ga[GSlab<BM, AKC, VEC>::PER], gb[GSlab<BN, BKC, VEC>::PER];
    la.load(ra, it0 * GEMM_BK, kend, ga);
    lb.load(rb, it0 * GEMM_BK, kend, gb);
    la.store(sA, ga);
    lb.store(sB, gb);
    la.load(ra, (it0 + 1) * GEMM_BK, kend, ga);
    lb.load(rb, (it0 + 1) * GEMM_BK, kend, gb);
    __syncthreads();
    read_frags(sA, sB, 0, f0a, f0b);
    for (int kt = it0; kt < it1; kt += 4) {
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int cur = u & 1;   // it0 is a multiple of 4: slab kt+u lives in buffer u & 1
            const float *ca = sA + cur * BM * G_LD, *cb = sB + cur * BN * G_LD;
            float *na = sA + (cur ^ 1) * BM * G_LD, *nb = sB + (cur ^ 1) * BN * G_LD;
            read_frags(ca, cb, 1, f1a, f1b);
            __builtin_amdgcn_sched_barrier(0);
            mfmas(f0a, f0b);
            __builtin_amdgcn_sched_barrier(0);
            la.store(na, ga);
            lb.store(nb, gb);
            __syncthreads();
            read_frags(na, nb, 0, f0a, f0b);
            __builtin_amdgcn_sched_barrier(0);
            la.load(ra, (kt + u + 2) * GEMM_BK, kend, ga);
            lb.load(rb, (kt + u + 2) * GEMM_BK, kend, gb);
            mfmas(f1a, f1b);
#pragma unroll
            for (int q = 0; q < NLOAD; ++q) {
                __builtin_amdgcn_sched_group_barrier(0x008, 4 * TM * TN / NLOAD, 0);   // MFMA
                __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);                   // VMEM read
            }
            __builtin_amdgcn_sched_barrier(0);
        }
#pragma unroll
        for (int a = 0; a < TM; ++a)
#pragma unroll
            for (int b = 0; b < TN; ++b) {
                tot[a][b] += acc[a][b];
                acc[a][b] = f4{0.f, 0.f, 0.f, 0.f};
            }
    }
    if (unit >= 0) {
        float *mine = p.ws + (int64_t)unit * (BM * BN);
#pragma unroll
        for (int a = 0; a < TM; ++a)
#pragma unroll
            for (int b = 0; b < TN; ++b) *(f4 *)(mine + ((a * TN + b) * GEMM_NT + tid) * 4) = tot[a][b];
        return;
    }
    g_epilogue<BM, BN, EPI>(p, tot, i0, j0, tid);
}

// The epilogue of one MFMA block (a, b) of a 64x64 tile: v holds output rows
// 4*lg + r of the block, column li (g_epilogue_act's coordinates).
template <int EPI, int ACT, bool IA, bool IB>
__device__ __forceinline__ void g_epilogue_blk_act(const GemmArgs &p, const f4 &v, int a, int b, int i0, int j0,
                                                   int tid) {
    const int lane = tid & 63, wave = tid >> 6, wm = wave >> 1, wn = wave & 1;
    const int li = lane & 15, lg = lane >> 4;
    int ii[4], jj[4];
    float vv[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int row = IA ? wm * 32 + 2 * (4 * lg + r) + a : wm * 32 + a * 16 + 4 * lg + r;
        const int col = IB ? wn * 32 + 2 * li + b : wn * 32 + b * 16 + li;
        ii[r] = i0 + row;
        jj[r] = j0 + col;
        vv[r] = v[r];
    }
    g_out_n<4, ACT, EPI>(p, ii, jj, vv);
}

// Sum of the segment partials of one MFMA block of a split 64x64 tile
// (blockIdx.x = 4 * tail + block), in segment order, then the block's
// epilogue.  A partial tile is stored as [block][thread][4] (the split
// kernels' write-back), so each thread reads one float4 per segment, and all
// of a thread's segment loads are issued before the first add: the launch
// is one round trip of latency, not one per segment.
#define FIXUP_MAX_SEGS 16
template <int EPI, bool IA, bool IB, bool DB, int SEL = SEL_NONE>
__device__ __forceinline__ void gemm_tile_fixup_body(const GemmArgs &pa) {
    const int tid = threadIdx.x, tail = blockIdx.x >> 2, blk = blockIdx.x & 3;
    int tm, tn;
    tile_rc<8>(pa.dp_tiles + tail, pa.tiles_m, pa.tiles_n, tm, tn);
    GemmArgs pl = pa;
    const int jb = SEL == SEL_F3 ? f3_select(pa, pl, tn * 64) : 0;
    if (SEL == SEL_HEADS) heads_select(pa, pl, tm * 64, tn * 64);
    const GemmArgs &p = SEL != SEL_NONE ? pl : pa;
    const float *first = p.ws + (int64_t)tail * p.segs * 4096 + (blk * GEMM_NT + tid) * 4;
    // unconditional loads (a segment index clamped to the last one, the extra
    // values not added): a guarded load is a branch with a wait after it
    f4 part[FIXUP_MAX_SEGS];
#pragma unroll
    for (int s = 0; s < FIXUP_MAX_SEGS; ++s) part[s] = *(const f4 *)(first + (int64_t)min(s, p.segs - 1) * 4096);
    f4 tot = part[0];
#pragma unroll
    for (int s = 1; s < FIXUP_MAX_SEGS; ++s) tot = s < p.segs ? tot + part[s] : tot;
    const int a = blk >> 1, b = blk & 1, i0 = tm * 64, j0 = tn * 64 - jb;
    if (EPI == EPI_ACCUM || EPI == EPI_ACT_BWD) {
        g_epilogue_blk_act<EPI, ACT_NONE, IA, IB>(p, tot, a, b, i0, j0, tid);
        // dW: the bias gradient of a split tile in tile column 0, from its
        // segments' fp64 partials in segment order
        if (DB && p.db != nullptr && tn == 0 && blk == 0 && tid < 64) {
            const double *q = p.dbpart + (int64_t)tail * p.segs * 64 + tid;
            double dp[FIXUP_MAX_SEGS];
#pragma unroll
            for (int s = 0; s < FIXUP_MAX_SEGS; ++s) dp[s] = q[(int64_t)min(s, p.segs - 1) * 64];
            const int i = min(i0 + tid, p.Mo - 1);
            const float old = p.db[i];
            double sum = dp[0];
#pragma unroll
            for (int s = 1; s < FIXUP_MAX_SEGS; ++s) sum = s < p.segs ? sum + dp[s] : sum;
            if (i0 + tid < p.Mo) p.db[i] = old + (0.0f + (float)sum);
        }
        return;
    }
    switch (p.act) {
    case ACT_SILU: g_epilogue_blk_act<EPI, ACT_SILU, IA, IB>(p, tot, a, b, i0, j0, tid); break;
    case ACT_GELU: g_epilogue_blk_act<EPI, ACT_GELU, IA, IB>(p, tot, a, b, i0, j0, tid); break;
    case ACT_GELU_TANH: g_epilogue_blk_act<EPI, ACT_GELU_TANH, IA, IB>(p, tot, a, b, i0, j0, tid); break;
    case ACT_RELU2: g_epilogue_blk_act<EPI, ACT_RELU2, IA, IB>(p, tot, a, b, i0, j0, tid); break;
    default: g_epilogue_blk_act<EPI, ACT_NONE, IA, IB>(p, tot, a, b, i0, j0, tid); break;
    }
}

// GATED epilogue of one wave's 32 rows (from r0) x 32 columns (from j0): the
// gate value, its bias and activation, times the up value plus its bias -- the
// float operations of linear_fwd_ep(act) followed by mul_fwd.
template <int ACT>
__device__ __forceinline__ void g_gated_out(const GemmArgs &p, const f4 (&g)[2][2], const f4 (&u)[2][2], int r0,
                                            int j0, int li, int lg) {
    // the biases of the thread's 4 columns loaded first (a stand-in address
    // when absent), then the in-bounds elements computed and stored
    const bool hb = p.bias != nullptr, hb2 = p.bias2 != nullptr;
    float bg[2], bu[2];
#pragma unroll
    for (int b = 0; b < 2; ++b) {
        const int j = min(j0 + b * 16 + li, p.No - 1);
        bg[b] = *(hb ? p.bias + j : p.C);
        bu[b] = *(hb2 ? p.bias2 + j : p.C);
    }
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int b = 0; b < 2; ++b)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int i = r0 + a * 16 + 4 * lg + r, j = j0 + b * 16 + li;
                if (i >= p.Mo || j >= p.No) continue;
                float vg = g[a][b][r], vu = u[a][b][r];
                if (hb) vg += bg[b];
                vg = ncm_act(vg, ACT);
                if (hb2) vu += bu[b];
                p.C[(int64_t)i * p.ldc + j] = vg * vu;
            }
}

// ---------------------------------------------------------------- GEMM, direct-to-LDS loads
// Two LDS stages of 16 KB: five workgroups share a CU.  Per slab: fragment
// reads of chunk 1, MFMAs of chunk 0, wait for this wave's loads of the next
// slab, barrier (every wave's loads have landed and every read of the
// current stage is done), fragment reads of the next slab's chunk 0, loads of
// the slab after next into the current stage, MFMAs of chunk 1.
template <bool V>
struct BoolTag {
    static constexpr bool value = V;
};

// DB: the dW kernel that also sums the bias gradient (p.db); SEL: per-tile
// output selection (f3_select, heads_select); TAIL: p.iters need not be a
// multiple of 4 -- the slabs of a partial last group that lie wholly past the
// range are skipped (a separate instance: the check in the unrolled k loop
// cost the other launches 1.4%).
template <bool AKC, bool BKC, int EPI, bool DB = false, int SEL = SEL_NONE, bool TAIL = false>
__device__ __forceinline__ void gemm_dma_body(const GemmArgs &pa) {
    __shared__ __attribute__((aligned(16))) float sm[2 * 2 * D_SLAB];   // [stage][A | B]
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1, li = lane & 15, lg = lane >> 4;

    int tile, it0, it1, unit = -1;
    {
        const int b = blockIdx.x;
        if (b < pa.dp_tiles) {
            tile = xcd_remap(b, pa.dp_tiles);
            it0 = 0;
            it1 = pa.iters;
        } else {
            const int ntail = (pa.tiles_m * pa.tiles_n - pa.dp_tiles) * pa.segs;
            const int j = b - pa.dp_tiles;
            unit = ((pa.dp_tiles & 7) == 0) ? xcd_remap(j, ntail) : j;
            const int tail = unit / pa.segs, seg = unit - tail * pa.segs;
            tile = pa.dp_tiles + tail;
            const int q4 = (pa.iters + (TAIL ? 3 : 0)) >> 2;
            it0 = (int)((int64_t)seg * q4 / pa.segs) * 4;
            it1 = (int)((int64_t)(seg + 1) * q4 / pa.segs) * 4;
            if (TAIL) it1 = min(it1, pa.iters);
        }
    }
    int tm, tn;
    tile_rc<8>(tile, pa.tiles_m, pa.tiles_n, tm, tn);
    GemmArgs pl = pa;
    const int jb = SEL == SEL_F3 ? f3_select(pa, pl, tn * 64) : 0;
    if (SEL == SEL_HEADS) heads_select(pa, pl, tm * 64, tn * 64);
    const GemmArgs &p = SEL != SEL_NONE ? pl : pa;
    // GATED: tile columns 0-31 are output columns j0 .. j0 + 31 of the gate
    // product, 32-63 the same columns of the up product; waves 0-1 load the
    // gate's B rows, waves 2-3 the up projection's
    const bool up_rows = EPI == EPI_GATED && wave >= 2;
    const int i0 = tm * 64, j0 = tn * (EPI == EPI_GATED ? 32 : 64) - jb;
    const int kend = min(p.K, it1 * GEMM_BK);
    const __amdgpu_buffer_rsrc_t ra = make_rsrc(p.A, p.a_bytes), rb = make_rsrc(up_rows ? p.B2 : p.B, p.b_bytes);
    DSlab<AKC> la;
    DSlab<BKC> lb;
    la.init(wave, lane, p.lda, i0, p.Mo, kend);
    lb.init(wave, lane, p.ldb, up_rows ? j0 - 32 : j0, p.No, kend);

    f4 acc[2][2], tot[2][2];
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int b = 0; b < 2; ++b) acc[a][b] = tot[a][b] = f4{0.f, 0.f, 0.f, 0.f};
    auto mfmas = [&](const float (&fa)[2][4], const float (&fb)[2][4]) {
#pragma unroll
        for (int s = 0; s < 4; ++s)
#pragma unroll
            for (int a = 0; a < 2; ++a)
#pragma unroll
                for (int b = 0; b < 2; ++b) acc[a][b] = mfma4(fa[a][s], fb[b][s], acc[a][b]);
    };
    // dW with the bias gradient (DB kernels): A(i,k) = dy[k][i], so the
    // tiles of tile column 0 also sum their A fragments over k, in fp64, for
    // the column sums of dy.  Lane (li, lg) of wave (wm, wn) holds rows
    // wm 32 + 2 li and 2 li + 1 (blocks t = 0, 1) and, of every 16-wide k
    // chunk, k rows 4 lg .. 4 lg + 3 (steps s); both waves of a wm read the
    // same fragments, so wave wn sums block t = wn, into one accumulator per
    // step (no dependent chain inside a chunk).  The fragments of slabs past
    // the segment's (or the matrix's) end are zeros.  Those tiles run their
    // own copy of the k loop, so no other tile (and no other kernel) carries
    // the work or a branch in it.
    const bool dsum = DB && p.db != nullptr && tn == 0;
    const bool wodd = __builtin_amdgcn_readfirstlane(wn) != 0;
    double ds[4] = {0.0, 0.0, 0.0, 0.0};
    float *const sA0 = sm, *const sB0 = sm + D_SLAB, *const sA1 = sm + 2 * D_SLAB, *const sB1 = sm + 3 * D_SLAB;

    float f0a[2][4], f0b[2][4], f1a[2][4], f1b[2][4];
    la.load(ra, sA0, wave, it0 * GEMM_BK, p.lda);
    lb.load(rb, sB0, wave, it0 * GEMM_BK, p.ldb);
    __builtin_amdgcn_s_waitcnt(0x0f70);   // vmcnt(0)
    __syncthreads();
    d_frags<AKC>(sA0, wm, li, lg, 0, f0a);
    d_frags<BKC>(sB0, wn, li, lg, 0, f0b);
    la.load(ra, sA1, wave, (it0 + 1) * GEMM_BK, p.lda);
    lb.load(rb, sB1, wave, (it0 + 1) * GEMM_BK, p.ldb);
    auto kloop = [&](auto ds_tag) {
        constexpr bool DS = decltype(ds_tag)::value;
        auto colsum = [&](const float (&fa)[2][4]) {
            if constexpr (DS) {
#pragma unroll
                for (int s = 0; s < 4; ++s) ds[s] += (double)(wodd ? fa[1][s] : fa[0][s]);
            }
        };
        for (int kt = it0; kt < it1; kt += 4) {
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                if constexpr (TAIL) {
                    if (kt + u >= it1) break;
                }
                // it0 is a multiple of 4: slab kt+u lives in stage u & 1
                float *const ca = (u & 1) ? sA1 : sA0, *const cb = (u & 1) ? sB1 : sB0;
                float *const na = (u & 1) ? sA0 : sA1, *const nb = (u & 1) ? sB0 : sB1;
                d_frags<AKC>(ca, wm, li, lg, 1, f1a);
                d_frags<BKC>(cb, wn, li, lg, 1, f1b);
                __builtin_amdgcn_sched_barrier(0);
                mfmas(f0a, f0b);
                colsum(f0a);
                __builtin_amdgcn_sched_barrier(0);
                __builtin_amdgcn_s_waitcnt(0x0f70);   // vmcnt(0): this wave's loads of slab kt+u+1
                __syncthreads();
                d_frags<AKC>(na, wm, li, lg, 0, f0a);
                d_frags<BKC>(nb, wn, li, lg, 0, f0b);
                __builtin_amdgcn_sched_barrier(0);
                la.load(ra, ca, wave, (kt + u + 2) * GEMM_BK, p.lda);
                lb.load(rb, cb, wave, (kt + u + 2) * GEMM_BK, p.ldb);
                __builtin_amdgcn_sched_barrier(0);
                mfmas(f1a, f1b);
                colsum(f1a);
                __builtin_amdgcn_sched_barrier(0);
            }
#pragma unroll
            for (int a = 0; a < 2; ++a)
#pragma unroll
                for (int b = 0; b < 2; ++b) {
                    tot[a][b] += acc[a][b];
                    acc[a][b] = f4{0.f, 0.f, 0.f, 0.f};
                }
        }
    };
    if (dsum)
        kloop(BoolTag<DB>{});
    else
        kloop(BoolTag<false>{});
    // No load may still be writing LDS when the workgroup ends.
    __builtin_amdgcn_s_waitcnt(0x0f70);
    if (dsum) {
        double d = (ds[0] + ds[1]) + (ds[2] + ds[3]);
        d += __shfl_xor(d, 16);
        d += __shfl_xor(d, 32);
        const int r = wm * 32 + 2 * li + wn;
        if (unit >= 0) {
            if (lg == 0) p.dbpart[(int64_t)unit * 64 + r] = d;
        } else if (lg == 0) {
            // a row past Mo reads the clamped address and writes nothing
            const int i = min(i0 + r, p.Mo - 1);
            const float old = p.db[i];
            if (i0 + r < p.Mo) p.db[i] = old + (0.0f + (float)d);
        }
    }
    if (unit >= 0) {
        float *mine = p.ws + (int64_t)unit * 4096;
#pragma unroll
        for (int a = 0; a < 2; ++a)
#pragma unroll
            for (int b = 0; b < 2; ++b) *(f4 *)(mine + ((a * 2 + b) * GEMM_NT + tid) * 4) = tot[a][b];
        return;
    }
    if constexpr (EPI == EPI_GATED) {
        // the up half (waves with wn = 1) hands its values to the gate half
        // through LDS: the same (a, b, lane) slot is the same output element
        __syncthreads();
        f4 *xch = (f4 *)sm;
        if (wn) {
#pragma unroll
            for (int a = 0; a < 2; ++a)
#pragma unroll
                for (int b = 0; b < 2; ++b) xch[((wm * 2 + a) * 2 + b) * 64 + lane] = tot[a][b];
        }
        __syncthreads();
        if (!wn) {
            f4 up[2][2];
#pragma unroll
            for (int a = 0; a < 2; ++a)
#pragma unroll
                for (int b = 0; b < 2; ++b) up[a][b] = xch[((wm * 2 + a) * 2 + b) * 64 + lane];
            switch (p.act) {
            case ACT_SILU: g_gated_out<ACT_SILU>(p, tot, up, i0 + wm * 32, j0, li, lg); break;
            case ACT_GELU: g_gated_out<ACT_GELU>(p, tot, up, i0 + wm * 32, j0, li, lg); break;
            case ACT_GELU_TANH: g_gated_out<ACT_GELU_TANH>(p, tot, up, i0 + wm * 32, j0, li, lg); break;
            case ACT_RELU2: g_gated_out<ACT_RELU2>(p, tot, up, i0 + wm * 32, j0, li, lg); break;
            default: g_gated_out<ACT_NONE>(p, tot, up, i0 + wm * 32, j0, li, lg); break;
            }
        }
        return;
    }
    g_epilogue<64, 64, EPI, !AKC, !BKC>(p, tot, i0, j0, tid);
}

// Register-staged kernels: four workgroups of 64x64 tiles share a CU (LDS), the register budget
// is held to that occupancy.  (128-wide tiles were measured slower on every
// linear-sweep shape: one or two workgroups per CU hide less latency.)
#define GEMM_TILE_KERNEL(name, BM, BN, AKC, BKC, EPI, VEC)                                          \
    extern "C" __global__ void __launch_bounds__(GEMM_NT)                                          \
        __attribute__((amdgpu_waves_per_eu(BM * BN <= 4096 ? 4 : 1))) name(GemmArgs p) {          \
        gemm_tile_body<BM, BN, AKC, BKC, EPI, VEC>(p);                                               \
    }
#define GEMM_DMA_KERNEL(name, AKC, BKC, EPI, DB, SEL)                                                   \
    extern "C" __global__ void __launch_bounds__(GEMM_NT) __attribute__((amdgpu_waves_per_eu(4)))      \
        name(GemmArgs p) {                                                                             \
        gemm_dma_body<AKC, BKC, EPI, DB, SEL>(p);                                                      \
    }
#define GEMM_DMA_TAIL_KERNEL(name, AKC, BKC, EPI, DB, SEL)                                              \
    extern "C" __global__ void __launch_bounds__(GEMM_NT) __attribute__((amdgpu_waves_per_eu(4)))      \
        name(GemmArgs p) {                                                                             \
        gemm_dma_body<AKC, BKC, EPI, DB, SEL, true>(p);                                                \
    }
#define GEMM_TILE_FIXUP(name, EPI, IA, IB, DB, SEL) \
    extern "C" __global__ void __launch_bounds__(GEMM_NT) name(GemmArgs p) { gemm_tile_fixup_body<EPI, IA, IB, DB, SEL>(p); }
GEMM_DMA_KERNEL(gemm_64x64_fwd_v, true, true, EPI_STORE, false, SEL_NONE)
GEMM_DMA_KERNEL(gemm_64x64_fwd3_v, true, true, EPI_STORE, false, SEL_F3)   // products side by side
GEMM_DMA_KERNEL(gemm_64x64_fwdh_v, true, true, EPI_STORE, false, SEL_HEADS)  // q | k | v to head-major
GEMM_DMA_KERNEL(gemm_64x64_dx_v, true, false, EPI_ACCUM, false, SEL_NONE)
GEMM_DMA_KERNEL(gemm_64x64_dw_v, false, false, EPI_ACCUM, false, SEL_NONE)
GEMM_DMA_KERNEL(gemm_64x64_dwb_v, false, false, EPI_ACCUM, true, SEL_NONE)   // dW + db
GEMM_DMA_TAIL_KERNEL(gemm_64x64_dwbt_v, false, false, EPI_ACCUM, true, SEL_NONE)   // dW + db, partial last group
GEMM_DMA_KERNEL(gemm_64x64_dxa_v, true, false, EPI_ACT_BWD, false, SEL_NONE) // dX through the activation backward
GEMM_DMA_KERNEL(gemm_64x64_dxh_v, true, false, EPI_ACCUM, false, SEL_HEADS)  // dX to head-major
GEMM_DMA_KERNEL(gemm_64x64_gated_v, true, true, EPI_GATED, false, SEL_NONE)
GEMM_TILE_KERNEL(gemm_64x64_fwd_s, 64, 64, true, true, EPI_STORE, false)
GEMM_TILE_KERNEL(gemm_64x64_dx_s, 64, 64, true, false, EPI_ACCUM, false)
GEMM_TILE_KERNEL(gemm_64x64_dw_s, 64, 64, false, false, EPI_ACCUM, false)
GEMM_TILE_FIXUP(gemm_64x64_fixup_fwd_v, EPI_STORE, false, false, false, SEL_NONE)
GEMM_TILE_FIXUP(gemm_64x64_fixup_fwd3_v, EPI_STORE, false, false, false, SEL_F3)
GEMM_TILE_FIXUP(gemm_64x64_fixup_fwdh_v, EPI_STORE, false, false, false, SEL_HEADS)
GEMM_TILE_FIXUP(gemm_64x64_fixup_dx_v, EPI_ACCUM, false, true, false, SEL_NONE)
GEMM_TILE_FIXUP(gemm_64x64_fixup_dw_v, EPI_ACCUM, true, true, false, SEL_NONE)
GEMM_TILE_FIXUP(gemm_64x64_fixup_dwb_v, EPI_ACCUM, true, true, true, SEL_NONE)
GEMM_TILE_FIXUP(gemm_64x64_fixup_dxa_v, EPI_ACT_BWD, false, true, false, SEL_NONE)
GEMM_TILE_FIXUP(gemm_64x64_fixup_dxh_v, EPI_ACCUM, false, true, false, SEL_HEADS)
GEMM_TILE_FIXUP(gemm_64x64_fixup_fwd_s, EPI_STORE, false, false, false, SEL_NONE)
GEMM_TILE_FIXUP(gemm_64x64_fixup_dx_s, EPI_ACCUM, false, false, false, SEL_NONE)
GEMM_TILE_FIXUP(gemm_64x64_fixup_dw_s, EPI_ACCUM, false, false, false, SEL_NONE)

// ---------------------------------------------------------------- GEMM, 128 x 128 tiles
// The direct-to-LDS pipeline of gemm_dma_body on 128 x 128 tiles: each wave
// owns a 64 x 64 sub-tile of 4 x 4 MFMA blocks, so a 16-wide chunk costs the
// wave 8 fragment reads for 64 MFMAs (4 for 16 on 64 x 64 tiles) and the
// operand traffic from L2 per FLOP halves.  Two stages of 32 KB: two
// workgroups share a CU.  Used where whole tiles fill the CUs (no split-K).
// The 128-row slabs and their fragment reads are mfma_slab.h's DSlabBig and
// d_frags_big.

// The epilogue of a 128 x 128 tile, one row of MFMA blocks (16 outputs per
// thread) at a time, so that the loaded operands of all 64 outputs are not
// live at once.
template <int EPI, int ACT, bool IA, bool IB>
__device__ __forceinline__ void g_epilogue_big_act(const GemmArgs &p, const f4 (&tot)[4][4], int i0, int j0,
                                                   int tid) {
    const int lane = tid & 63, wave = tid >> 6, wm = wave >> 1, wn = wave & 1;
    const int li = lane & 15, lg = lane >> 4;
#pragma unroll
    for (int a = 0; a < 4; ++a) {
        int ii[16], jj[16];
        float v[16];
#pragma unroll
        for (int b = 0; b < 4; ++b)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int n = b * 4 + r;
                ii[n] = i0 + (IA ? wm * 64 + 4 * (4 * lg + r) + a : wm * 64 + a * 16 + 4 * lg + r);
                jj[n] = j0 + (IB ? wn * 64 + 4 * li + b : wn * 64 + b * 16 + li);
                v[n] = tot[a][b][r];
            }
        g_out_n<16, ACT, EPI>(p, ii, jj, v);
    }
}

template <int EPI, bool IA, bool IB>
__device__ __forceinline__ void g_epilogue_big(const GemmArgs &p, const f4 (&tot)[4][4], int i0, int j0, int tid) {
    if (EPI == EPI_ACCUM || EPI == EPI_ACT_BWD) {
        g_epilogue_big_act<EPI, ACT_NONE, IA, IB>(p, tot, i0, j0, tid);
        return;
    }
    switch (p.act) {
    case ACT_SILU: g_epilogue_big_act<EPI, ACT_SILU, IA, IB>(p, tot, i0, j0, tid); break;
    case ACT_GELU: g_epilogue_big_act<EPI, ACT_GELU, IA, IB>(p, tot, i0, j0, tid); break;
    case ACT_GELU_TANH: g_epilogue_big_act<EPI, ACT_GELU_TANH, IA, IB>(p, tot, i0, j0, tid); break;
    case ACT_RELU2: g_epilogue_big_act<EPI, ACT_RELU2, IA, IB>(p, tot, i0, j0, tid); break;
    default: g_epilogue_big_act<EPI, ACT_NONE, IA, IB>(p, tot, i0, j0, tid); break;
    }
}

// Whole 128 x 128 tiles (blockIdx.x = tile; dp_tiles = all tiles).  DB: the
// dW kernel that also sums the bias gradient; SEL_HEADS: each wave's 64
// output columns lie in one head and its 128 rows in one sequence (T a
// multiple of 128), so the wave stores into that head's [128 t][64 d] block.
template <bool AKC, bool BKC, int EPI, bool DB = false, int SEL = SEL_NONE>
__device__ __forceinline__ void gemm_big_body(const GemmArgs &pa) {
    __shared__ __attribute__((aligned(16))) float sm[2 * 2 * D_SLAB_BIG];   // [stage][A | B]
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1, li = lane & 15, lg = lane >> 4;
    const int tile = xcd_remap(blockIdx.x, pa.tiles_m * pa.tiles_n);
    int tm, tn;
    tile_rc<8>(tile, pa.tiles_m, pa.tiles_n, tm, tn);
    const int i0 = tm * BIG, j0 = tn * BIG;
    GemmArgs pl = pa;
    if (SEL == SEL_HEADS) heads_select(pa, pl, i0, j0 + wn * 64);
    const GemmArgs &p = SEL != SEL_NONE ? pl : pa;
    const int kend = p.K;
    const __amdgpu_buffer_rsrc_t ra = make_rsrc(p.A, p.a_bytes), rb = make_rsrc(p.B, p.b_bytes);
    DSlabBig<AKC> la;
    DSlabBig<BKC> lb;
    la.init(wave, lane, p.lda, i0, p.Mo, kend);
    lb.init(wave, lane, p.ldb, j0, p.No, kend);

    f4 acc[4][4], tot[4][4];
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int b = 0; b < 4; ++b) acc[a][b] = tot[a][b] = f4{0.f, 0.f, 0.f, 0.f};
    auto mfmas = [&](const float (&fa)[4][4], const float (&fb)[4][4]) {
#pragma unroll
        for (int s = 0; s < 4; ++s)
#pragma unroll
            for (int a = 0; a < 4; ++a)
#pragma unroll
                for (int b = 0; b < 4; ++b) acc[a][b] = mfma4(fa[a][s], fb[b][s], acc[a][b]);
    };
    // dW with the bias gradient: A(i,k) = dy[k][i], so the tiles of tile
    // column 0 also sum each A slab over k in fp64, straight from LDS while
    // the slab is current: thread t takes tile row t & 127 and the slab's k
    // rows 16 (t >> 7) .. + 15 (consecutive lanes, consecutive banks); the
    // two halves are added at the end.  (Summing the MFMA fragments in
    // registers, as the 64 x 64 kernel does, spilled at this tile size.)
    const bool dsum = DB && p.db != nullptr && tn == 0;
    double ds = 0.0;
    float *const sA0 = sm, *const sB0 = sm + D_SLAB_BIG, *const sA1 = sm + 2 * D_SLAB_BIG,
                 *const sB1 = sm + 3 * D_SLAB_BIG;
    const int iters = p.iters;

    float f0a[4][4], f0b[4][4], f1a[4][4], f1b[4][4];
    la.load(ra, sA0, wave, 0, p.lda);
    lb.load(rb, sB0, wave, 0, p.ldb);
    __builtin_amdgcn_s_waitcnt(0x0f70);   // vmcnt(0)
    __syncthreads();
    d_frags_big<AKC>(sA0, wm, li, lg, 0, f0a);
    d_frags_big<BKC>(sB0, wn, li, lg, 0, f0b);
    la.load(ra, sA1, wave, GEMM_BK, p.lda);
    lb.load(rb, sB1, wave, GEMM_BK, p.ldb);
    auto kloop = [&](auto ds_tag) {
        constexpr bool DS = decltype(ds_tag)::value;
        auto colsum = [&](const float *slab) {
            if constexpr (DS) {
                const float *q = slab + 16 * (tid >> 7) * BIG + (tid & 127);
#pragma unroll
                for (int k = 0; k < 16; ++k) ds += (double)q[k * BIG];
            }
        };
        for (int kt = 0; kt < iters; kt += 4) {
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                float *const ca = (u & 1) ? sA1 : sA0, *const cb = (u & 1) ? sB1 : sB0;
                float *const na = (u & 1) ? sA0 : sA1, *const nb = (u & 1) ? sB0 : sB1;
                d_frags_big<AKC>(ca, wm, li, lg, 1, f1a);
                d_frags_big<BKC>(cb, wn, li, lg, 1, f1b);
                colsum(ca);
                __builtin_amdgcn_sched_barrier(0);
                mfmas(f0a, f0b);
                __builtin_amdgcn_sched_barrier(0);
                __builtin_amdgcn_s_waitcnt(0x0f70);   // vmcnt(0): this wave's loads of slab kt+u+1
                __syncthreads();
                d_frags_big<AKC>(na, wm, li, lg, 0, f0a);
                d_frags_big<BKC>(nb, wn, li, lg, 0, f0b);
                __builtin_amdgcn_sched_barrier(0);
                la.load(ra, ca, wave, (kt + u + 2) * GEMM_BK, p.lda);
                lb.load(rb, cb, wave, (kt + u + 2) * GEMM_BK, p.ldb);
                __builtin_amdgcn_sched_barrier(0);
                mfmas(f1a, f1b);
                __builtin_amdgcn_sched_barrier(0);
            }
#pragma unroll
            for (int a = 0; a < 4; ++a)
#pragma unroll
                for (int b = 0; b < 4; ++b) {
                    tot[a][b] += acc[a][b];
                    acc[a][b] = f4{0.f, 0.f, 0.f, 0.f};
                }
        }
    };
    if (dsum)
        kloop(BoolTag<DB>{});
    else
        kloop(BoolTag<false>{});
    // No load may still be writing LDS when the workgroup ends.
    __builtin_amdgcn_s_waitcnt(0x0f70);
    if (dsum) {
        __syncthreads();   // every wave is done with the slabs: reuse the LDS
        double *half = (double *)sm;
        if (tid >= 128) half[tid - 128] = ds;
        __syncthreads();
        if (tid < 128) {
            // a row past Mo reads the clamped address and writes nothing
            const double d = ds + half[tid];
            const int i = min(i0 + tid, p.Mo - 1);
            const float old = p.db[i];
            if (i0 + tid < p.Mo) p.db[i] = old + (0.0f + (float)d);
        }
    }
    g_epilogue_big<EPI, !AKC, !BKC>(p, tot, i0, j0, tid);
}

#define GEMM_BIG_KERNEL(name, AKC, BKC, EPI, DB, SEL)                                                   \
    extern "C" __global__ void __launch_bounds__(GEMM_NT) __attribute__((amdgpu_waves_per_eu(2)))      \
        name(GemmArgs p) {                                                                             \
        gemm_big_body<AKC, BKC, EPI, DB, SEL>(p);                                                      \
    }
GEMM_BIG_KERNEL(gemm_128x128_fwd_v, true, true, EPI_STORE, false, SEL_NONE)
GEMM_BIG_KERNEL(gemm_128x128_fwdh_v, true, true, EPI_STORE, false, SEL_HEADS)
GEMM_BIG_KERNEL(gemm_128x128_dx_v, true, false, EPI_ACCUM, false, SEL_NONE)
GEMM_BIG_KERNEL(gemm_128x128_dw_v, false, false, EPI_ACCUM, false, SEL_NONE)
GEMM_BIG_KERNEL(gemm_128x128_dwb_v, false, false, EPI_ACCUM, true, SEL_NONE)
GEMM_BIG_KERNEL(gemm_128x128_dxa_v, true, false, EPI_ACT_BWD, false, SEL_NONE)
GEMM_BIG_KERNEL(gemm_128x128_dxh_v, true, false, EPI_ACCUM, false, SEL_HEADS)
