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
// Tiling: a 256-thread workgroup owns a 128x128 output tile; each of its four
// 64-lane waves owns a 64x64 sub-tile of 4x4 MFMA blocks.  Operand slabs of
// BK = 32 go global -> registers -> LDS (two LDS buffers) and are consumed as
// two 16-wide chunks.  Per slab and wave (128 MFMAs):
//   chunk 0 MFMAs, interleaved with: LDS reads of chunk 1, LDS writes of the
//       next slab (other buffer), global loads of the slab after next;
//   one barrier;
//   chunk 1 MFMAs, interleaved with the LDS reads of the next slab's chunk 0.
// The interleaving is imposed with scheduling-group barriers, so the matrix
// pipe keeps issuing while the memory traffic is in flight.  Global loads are
// raw buffer loads: lanes outside the matrix get an offset beyond the buffer
// and read zero, so the loop body has no branches.
//
// k-permutation: inside every 16-wide chunk, MFMA step s (0..3) gives lane
// group g = lane/16 the reduction index k = 4g + s, for both operands.  The
// MFMA sums over all 16 (g, s) pairs, so the product is unchanged, but every
// operand read becomes a 128-bit LDS load:
//   k-contiguous operand : one float4 along k per lane covers all 4 steps;
//   i/j-contiguous operand: one float4 along i/j per lane and step covers 4
//                           MFMA blocks whose rows (cols) interleave with
//                           stride 4 (block u of a 64-wide group holds rows
//                           4*lane16 + u).
//
// Scheduling: tiles [0, dp_tiles) run whole, one workgroup each; every other
// tile is cut into `segs` k-segments that fill the last round of the chip.
// Segments store partial tiles; gemm_fixup (a second launch) sums them in
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
    float *ws;           // partial tiles of split tiles [units][BM*BN]
    int Mo, No, K;
    int lda, ldb, ldc;
    int act;
    int vec_out;         // output rows 16-byte aligned and No % 4 == 0
    int tiles_m, tiles_n;
    int iters;           // BK slabs per tile (a multiple of 4)
    int dp_tiles;        // blocks [0, dp_tiles): one whole tile each
    int segs;            // later blocks: k-segment (u % segs) of tile dp_tiles + u / segs
    unsigned a_bytes, b_bytes;  // extents of A and B for the buffer descriptors
};

#define GEMM_BM 128
#define GEMM_BN 128
#define GEMM_BK 32
#define GEMM_NT 256
#define OOB_OFFSET 0x80000000u
#ifndef GEMM_LDS_PAD
#define GEMM_LDS_PAD 8   // floats of padding per LDS tile row: a 40-float pitch makes the
                         // k-contiguous fragment reads (16 rows x 16 B per 16 lanes) hit all 64 banks
#endif

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

// One operand tile of ROWS x COLS floats per slab, as laid out in memory
// (row stride ld); the slab index moves along columns (KALONG_COLS) or rows.
// Thread t owns the float4s f = t + j*NT (j < PER): since NT is a multiple
// of the float4s per row, all of them share one column and sit RSTEP rows
// apart, so the whole per-thread state is three registers.
template <int ROWS, int COLS, bool KALONG_COLS, bool VEC>
struct SlabLoader {
    static constexpr int F4 = ROWS * COLS / 4;
    static constexpr int PER = F4 / GEMM_NT;
    static constexpr int RSTEP = GEMM_NT / (COLS / 4);
    static_assert(F4 % GEMM_NT == 0 && GEMM_NT % (COLS / 4) == 0, "tile must split evenly");
    int row0, col0;        // global row / column of this thread's first float4 (slab 0)
    int lds0;              // LDS float offset of that float4
    f4 r[PER];

    __device__ __forceinline__ void init(int fix0, int k0, int tid) {
        const int rr = tid / (COLS / 4), cc = (tid % (COLS / 4)) * 4;
        lds0 = rr * (COLS + GEMM_LDS_PAD) + cc;
        row0 = (KALONG_COLS ? fix0 : k0) + rr;
        col0 = (KALONG_COLS ? k0 : fix0) + cc;
    }

    // slab kt (k advanced by kt*BK); rows >= row_lim / columns >= col_lim read zero
    __device__ __forceinline__ void load(__amdgpu_buffer_rsrc_t rs, int ld, int kt, int row_lim, int col_lim) {
        const int dk = kt * GEMM_BK;
        const int c = col0 + (KALONG_COLS ? dk : 0);
#pragma unroll
        for (int j = 0; j < PER; ++j) {
            const int rw = row0 + j * RSTEP + (KALONG_COLS ? 0 : dk);
            const unsigned o = (unsigned)(rw * ld + c) * 4u;
            if (VEC) {
                const unsigned oo = (rw < row_lim && c < col_lim) ? o : OOB_OFFSET;
                r[j] = __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(rs, oo, 0, 0));
            } else {
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    const unsigned oo = (rw < row_lim && c + u < col_lim) ? o + 4u * u : OOB_OFFSET;
                    r[j][u] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs, oo, 0, 0));
                }
            }
        }
    }

    __device__ __forceinline__ void store(float *buf) const {
#pragma unroll
        for (int j = 0; j < PER; ++j) *(f4 *)(buf + lds0 + j * RSTEP * (COLS + GEMM_LDS_PAD)) = r[j];
    }
};

// Epilogue of one tile from the per-thread accumulators.  tot[a][b][r] holds
// MFMA row rho = 4*lg + r, column gamma = li.
template <int TM, int TN, int WM, int WN, bool AKC, bool BKC, int EPI, int ACT>
__device__ __forceinline__ void gemm_epilogue_act(const GemmArgs &p, const f4 (&tot)[TM][TN], int i0, int j0, int tid,
                                                  int a_lo, int a_hi) {
    const int lane = tid & 63, wave = tid >> 6;
    const int wm = wave / (GEMM_BN / WN), wn = wave % (GEMM_BN / WN);
    const int li = lane & 15, lg = lane >> 4;
#pragma unroll
    for (int a = 0; a < TM; ++a) {
        if (a < a_lo || a >= a_hi) continue;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int rho = 4 * lg + r;
            const int row = i0 + wm * WM + (AKC ? a * 16 + rho : (a >> 2) * 64 + 4 * rho + (a & 3));
            if (row >= p.Mo) continue;
            float *orow = p.C + (int64_t)row * p.ldc;
            const float *rrow = (EPI == EPI_STORE && p.res) ? p.res + (int64_t)row * p.ldc : nullptr;
            if (!BKC && p.vec_out) {
                // the four blocks b = 4q+u hold columns 4*li + u: one float4 per q
#pragma unroll
                for (int q = 0; q < TN / 4; ++q) {
                    const int col = j0 + wn * WN + q * 64 + 4 * li;
                    if (col >= p.No) continue;
                    f4 v = {tot[a][4 * q][r], tot[a][4 * q + 1][r], tot[a][4 * q + 2][r], tot[a][4 * q + 3][r]};
                    f4 *o = (f4 *)(orow + col);
                    if (EPI == EPI_ACCUM) v += *o;
                    *o = v;
                }
                continue;
            }
#pragma unroll
            for (int b = 0; b < TN; ++b) {
                const int col = j0 + wn * WN + (BKC ? b * 16 + li : (b >> 2) * 64 + 4 * li + (b & 3));
                if (col >= p.No) continue;
                float v = tot[a][b][r];
                if (EPI == EPI_STORE) {
                    if (p.bias) v += p.bias[col];
                    v = ncm_act(v, ACT);
                    if (rrow) v = rrow[col] + v;
                    orow[col] = v;
                } else {
                    orow[col] += v;
                }
            }
        }
    }
}

// The activation is dispatched once per tile, so every instantiation is a
// short straight-line epilogue.
template <int TM, int TN, int WM, int WN, bool AKC, bool BKC, int EPI>
__device__ __forceinline__ void gemm_epilogue(const GemmArgs &p, const f4 (&tot)[TM][TN], int i0, int j0, int tid,
                                              int a_lo = 0, int a_hi = TM) {
    if (EPI == EPI_ACCUM) {
        gemm_epilogue_act<TM, TN, WM, WN, AKC, BKC, EPI, ACT_NONE>(p, tot, i0, j0, tid, a_lo, a_hi);
        return;
    }
    switch (p.act) {
    case ACT_SILU: gemm_epilogue_act<TM, TN, WM, WN, AKC, BKC, EPI, ACT_SILU>(p, tot, i0, j0, tid, a_lo, a_hi); break;
    case ACT_GELU: gemm_epilogue_act<TM, TN, WM, WN, AKC, BKC, EPI, ACT_GELU>(p, tot, i0, j0, tid, a_lo, a_hi); break;
    case ACT_GELU_TANH: gemm_epilogue_act<TM, TN, WM, WN, AKC, BKC, EPI, ACT_GELU_TANH>(p, tot, i0, j0, tid, a_lo, a_hi); break;
    default: gemm_epilogue_act<TM, TN, WM, WN, AKC, BKC, EPI, ACT_NONE>(p, tot, i0, j0, tid, a_lo, a_hi); break;
    }
}

template <bool AKC, bool BKC, int EPI, bool VEC>
__device__ __forceinline__ void gemm_body(const GemmArgs &p) {
    constexpr int BM = GEMM_BM, BN = GEMM_BN, BK = GEMM_BK, WM = 64, WN = 64;
    constexpr int WAVES_N = BN / WN;
    constexpr int TM = WM / 16, TN = WN / 16;
    constexpr int A_ROWS = AKC ? BM : BK, A_COLS = AKC ? BK : BM;
    constexpr int B_ROWS = BKC ? BN : BK, B_COLS = BKC ? BK : BN;
    constexpr int A_LD = A_COLS + GEMM_LDS_PAD, B_LD = B_COLS + GEMM_LDS_PAD;
    constexpr int A_SZ = A_ROWS * A_LD, B_SZ = B_ROWS * B_LD;
    __shared__ __attribute__((aligned(16))) float smem[2 * (A_SZ + B_SZ)];
    float *const sA = smem;               // buffers sA + {0, A_SZ}
    float *const sB = smem + 2 * A_SZ;    // buffers sB + {0, B_SZ}

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int wm = wave / WAVES_N, wn = wave % WAVES_N;
    const int li = lane & 15, lg = lane >> 4;

    // ---- which tile and which k-range ----
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
            const int tail = unit / p.segs;
            const int seg = unit - tail * p.segs;
            tile = p.dp_tiles + tail;
            // segment boundaries on multiples of 4 slabs
            const int q4 = p.iters >> 2;
            it0 = (int)((int64_t)seg * q4 / p.segs) * 4;
            it1 = (int)((int64_t)(seg + 1) * q4 / p.segs) * 4;
        }
    }
    int tm, tn;
    tile_rc<8>(tile, p.tiles_m, p.tiles_n, tm, tn);
    const int i0 = tm * BM, j0 = tn * BN;
    const int nk = it1 - it0;               // multiple of 4
    const int kend = min(p.K, it1 * BK);

    const __amdgpu_buffer_rsrc_t ra = make_rsrc(p.A, p.a_bytes);
    const __amdgpu_buffer_rsrc_t rb = make_rsrc(p.B, p.b_bytes);
    SlabLoader<A_ROWS, A_COLS, AKC, VEC> la;
    SlabLoader<B_ROWS, B_COLS, BKC, VEC> lb;
    la.init(i0, it0 * BK, tid);
    lb.init(j0, it0 * BK, tid);
    // bounds: (rows, cols) of A and B as stored
    const int a_rl = AKC ? p.Mo : kend, a_cl = AKC ? kend : p.Mo;
    const int b_rl = BKC ? p.No : kend, b_cl = BKC ? kend : p.No;

    // Fragments of one 16-wide chunk.  k-contiguous: f[t] = row block t,
    // component = MFMA step.  i-contiguous: f[s * TM/4 + q] = step s, group q,
    // component = row block 4q + u.  Same for B.
    auto frags = [&](const float *a_s, const float *b_s, int kc, f4 *fa, f4 *fb) {
        if (AKC) {
#pragma unroll
            for (int t = 0; t < TM; ++t)
                fa[t] = *(const f4 *)(a_s + (wm * WM + t * 16 + li) * A_LD + kc * 16 + 4 * lg);
        } else {
#pragma unroll
            for (int s = 0; s < 4; ++s)
#pragma unroll
                for (int q = 0; q < TM / 4; ++q)
                    fa[s * (TM / 4) + q] = *(const f4 *)(a_s + (kc * 16 + 4 * lg + s) * A_LD + wm * WM + q * 64 + 4 * li);
        }
        if (BKC) {
#pragma unroll
            for (int t = 0; t < TN; ++t)
                fb[t] = *(const f4 *)(b_s + (wn * WN + t * 16 + li) * B_LD + kc * 16 + 4 * lg);
        } else {
#pragma unroll
            for (int s = 0; s < 4; ++s)
#pragma unroll
                for (int q = 0; q < TN / 4; ++q)
                    fb[s * (TN / 4) + q] = *(const f4 *)(b_s + (kc * 16 + 4 * lg + s) * B_LD + wn * WN + q * 64 + 4 * li);
        }
    };

    f4 acc[TM][TN], tot[TM][TN];
#pragma unroll
    for (int a = 0; a < TM; ++a)
#pragma unroll
        for (int b = 0; b < TN; ++b) acc[a][b] = tot[a][b] = f4{0.f, 0.f, 0.f, 0.f};

    auto mfmas = [&](const f4 *fa, const f4 *fb) {
#pragma unroll
        for (int s = 0; s < 4; ++s)
#pragma unroll
            for (int a = 0; a < TM; ++a) {
                const float av = AKC ? fa[a][s] : fa[s * (TM / 4) + (a >> 2)][a & 3];
#pragma unroll
                for (int b = 0; b < TN; ++b) {
                    const float bv = BKC ? fb[b][s] : fb[s * (TN / 4) + (b >> 2)][b & 3];
                    acc[a][b] = mfma4(av, bv, acc[a][b]);
                }
            }
    };

    // prologue: slab 0 -> LDS buffer 0, slab 1 in registers, chunk 0 fragments
    f4 fa0[TM], fb0[TN], fa1[TM], fb1[TN];
    la.load(ra, p.lda, 0, a_rl, a_cl);
    lb.load(rb, p.ldb, 0, b_rl, b_cl);
    la.store(sA);
    lb.store(sB);
    la.load(ra, p.lda, 1, a_rl, a_cl);
    lb.load(rb, p.ldb, 1, b_rl, b_cl);
    __syncthreads();
    frags(sA, sB, 0, fa0, fb0);

    // slab kt lives in buffer kt&1; slabs >= nk read zeros and are never used
    auto slab = [&](int kt, const int cur) {
        const float *a_s = sA + cur * A_SZ, *b_s = sB + cur * B_SZ;
        // chunk 0 MFMAs || chunk 1 fragments, next slab -> other buffer, slab kt+2 loads
        frags(a_s, b_s, 1, fa1, fb1);
        la.store(sA + (cur ^ 1) * A_SZ);
        lb.store(sB + (cur ^ 1) * B_SZ);
        la.load(ra, p.lda, kt + 2, a_rl, a_cl);
        lb.load(rb, p.ldb, kt + 2, b_rl, b_cl);
        mfmas(fa0, fb0);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);   // 2 LDS reads
            __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);   // 2 MFMA
            __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);   // 1 LDS write
            __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
            __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);   // 1 global load
            __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);
        }
        __syncthreads();
        // chunk 1 MFMAs || next slab's chunk 0 fragments
        frags(sA + (cur ^ 1) * A_SZ, sB + (cur ^ 1) * B_SZ, 0, fa0, fb0);
        mfmas(fa1, fb1);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 1);
            __builtin_amdgcn_sched_group_barrier(0x008, 8, 1);
        }
    };

    for (int kt = 0; kt < nk; kt += 4) {
        slab(kt, 0);
        slab(kt + 1, 1);
        slab(kt + 2, 0);
        slab(kt + 3, 1);
#pragma unroll
        for (int a = 0; a < TM; ++a)
#pragma unroll
            for (int b = 0; b < TN; ++b) {
                tot[a][b] += acc[a][b];
                acc[a][b] = f4{0.f, 0.f, 0.f, 0.f};
            }
    }

    if (unit >= 0) {
        // split tile: publish the partial; gemm_fixup finishes the tile
        float *mine = p.ws + (int64_t)unit * (BM * BN);
#pragma unroll
        for (int a = 0; a < TM; ++a)
#pragma unroll
            for (int b = 0; b < TN; ++b) *(f4 *)(mine + ((a * TN + b) * GEMM_NT + tid) * 4) = tot[a][b];
        return;
    }
    gemm_epilogue<TM, TN, WM, WN, AKC, BKC, EPI>(p, tot, i0, j0, tid);
}

// Sum of the segment partials of split tile blockIdx.x in segment order,
// then the epilogue (same thread -> element mapping as gemm_body).  Each
// workgroup finishes one of the TM row blocks (blockIdx.y), so a tile's
// partials are read by TM CUs in parallel.
template <bool AKC, bool BKC, int EPI>
__device__ __forceinline__ void gemm_fixup_body(const GemmArgs &p) {
    constexpr int TM = 4, TN = 4;
    const int tid = threadIdx.x;
    const int tail = blockIdx.x;
    const int a0 = blockIdx.y;
    int tm, tn;
    tile_rc<8>(p.dp_tiles + tail, p.tiles_m, p.tiles_n, tm, tn);
    const float *first = p.ws + (int64_t)tail * p.segs * (GEMM_BM * GEMM_BN);
    f4 tot[TM][TN];
#pragma unroll
    for (int a = 0; a < TM; ++a)
#pragma unroll
        for (int b = 0; b < TN; ++b) tot[a][b] = f4{0.f, 0.f, 0.f, 0.f};
    for (int sg = 0; sg < p.segs; ++sg) {
        const f4 *src = (const f4 *)(first + (int64_t)sg * (GEMM_BM * GEMM_BN));
#pragma unroll
        for (int a = 0; a < TM; ++a) {
            if (a != a0) continue;
#pragma unroll
            for (int b = 0; b < TN; ++b) tot[a][b] += __builtin_nontemporal_load(src + (a * TN + b) * GEMM_NT + tid);
        }
    }
    gemm_epilogue<TM, TN, 64, 64, AKC, BKC, EPI>(p, tot, tm * GEMM_BM, tn * GEMM_BN, tid, a0, a0 + 1);
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
#define GEMM_KERNEL(name, AKC, BKC, EPI, VEC)                                                  \
    extern "C" __global__ void __launch_bounds__(GEMM_NT, 1) name(GemmArgs p) {                \
        gemm_body<AKC, BKC, EPI, VEC>(p);                                                      \
    }
#define FIXUP_KERNEL(name, AKC, BKC, EPI)                                                      \
    extern "C" __global__ void __launch_bounds__(GEMM_NT) name(GemmArgs p) {                   \
        gemm_fixup_body<AKC, BKC, EPI>(p);                                                     \
    }

GEMM_KERNEL(gemm_fwd_v, true,  true,  EPI_STORE, true)
GEMM_KERNEL(gemm_fwd_s, true,  true,  EPI_STORE, false)
GEMM_KERNEL(gemm_dx_v,  true,  false, EPI_ACCUM, true)
GEMM_KERNEL(gemm_dx_s,  true,  false, EPI_ACCUM, false)
GEMM_KERNEL(gemm_dw_v,  false, false, EPI_ACCUM, true)
GEMM_KERNEL(gemm_dw_s,  false, false, EPI_ACCUM, false)
FIXUP_KERNEL(gemm_fixup_fwd, true,  true,  EPI_STORE)
FIXUP_KERNEL(gemm_fixup_dx,  true,  false, EPI_ACCUM)
FIXUP_KERNEL(gemm_fixup_dw,  false, false, EPI_ACCUM)

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
