// ncp.hip -- device pieces of the multi-level NCP forward (ncp.c:94-640 of
// the reference): the q/k/v split with qk-norm and RoPE, additive masks
// from the level layout, row gathers, per-level logits placement and the
// codebook-tied head.  Each repeats the reference's float operations for
// its values (RMSNorm's fp64 sum excepted, as everywhere in this library).
#include "ncm_dev.h"

// q [B][H][S][hd], k and v [B][nkv][S][hd] from qkv rows [B*S][C + 2 nkv hd]
// (ncp.c:206-244): one wave per output row, lane d holds element d (hd <= 64,
// even).  q and k rows are RMS-normalised with qn / kn when given
// (rmsnorm_fwd's arithmetic: fp64 mean of squares, s = (float)(1 /
// sqrt(ms + 1e-6)), y = (x s) w) and then rotated with table row s when cos_t
// is given (rope_one_exact: y[d] = a c[d] + (-b) s[d], y[d + h] = b c[d + h] +
// a s[d + h] for the pair (a, b) = (x[d], x[d + h])).
extern "C" __global__ void __launch_bounds__(256)
ncp_qkv_k(const float *__restrict__ qkv, float *__restrict__ q, float *__restrict__ k, float *__restrict__ v,
          const float *__restrict__ qn, const float *__restrict__ kn, const float *__restrict__ cos_t,
          const float *__restrict__ sin_t, int B, int S, int H, int nkv, int hd) {
#pragma clang fp contract(off)
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);   // over B * (H + 2 nkv) * S
    const int slots = H + 2 * nkv;
    if (row >= (int64_t)B * slots * S) return;
    const int s = (int)(row % S);
    const int slot = (int)((row / S) % slots);
    const int b = (int)(row / ((int64_t)S * slots));
    const int C = H * hd, W = C + 2 * nkv * hd;
    const float *src = qkv + ((int64_t)b * S + s) * W + (int64_t)slot * hd;   // q | k | v heads in order
    float *dst;
    const float *nw = nullptr;
    if (slot < H) {
        dst = q + (((int64_t)b * H + slot) * S + s) * hd;
        nw = qn;
    } else if (slot < H + nkv) {
        dst = k + (((int64_t)b * nkv + (slot - H)) * S + s) * hd;
        nw = kn;
    } else {
        dst = v + (((int64_t)b * nkv + (slot - H - nkv)) * S + s) * hd;
    }
    const bool act = lane < hd;
    float x = act ? src[lane] : 0.f;
    if (slot < H + nkv) {
        if (nw) {
            double ms = act ? (double)x * (double)x : 0.0;
            ms = wave_sum_d(ms) / hd;
            const float sc = (float)(1.0 / sqrt(ms + 1e-6));
            x = act ? x * sc * nw[lane] : 0.f;
        }
        if (cos_t) {
            const int h = hd >> 1;
            const float other = __shfl(x, lane < h ? lane + h : lane - h, 64);
            const float c = act ? cos_t[(int64_t)s * hd + lane] : 0.f;
            const float sn = act ? sin_t[(int64_t)s * hd + lane] : 0.f;
            x = lane < h ? x * c + (-other) * sn : x * c + other * sn;
        }
    }
    if (act) dst[lane] = x;
}

// The same for hd = 64 and H + 2 nkv <= 16 heads per row: one wave per qkv
// row (lane = d), the row's head loads all issued first (the slot index
// clamped; absent norm weights and tables read a stand-in address and are not
// used), row and head indices in 32-bit.  The per-head kernel's 64-bit
// division and one guarded round trip per head were most of its time.
extern "C" __global__ void __launch_bounds__(256)
ncp_qkv_rows_k(const float *__restrict__ qkv, float *__restrict__ q, float *__restrict__ k, float *__restrict__ v,
               const float *__restrict__ qn, const float *__restrict__ kn, const float *__restrict__ cos_t,
               const float *__restrict__ sin_t, int B, int S, int H, int nkv) {
#pragma clang fp contract(off)
    const int lane = threadIdx.x & 63, row = blockIdx.x * 4 + (threadIdx.x >> 6);   // row = b S + s
    if (row >= B * S) return;
    const int b = row / S, s = row - b * S, slots = H + 2 * nkv;
    const float *src = qkv + (int64_t)row * slots * 64 + lane;
    float xv[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) xv[j] = src[min(j, slots - 1) * 64];
    const float wq = *(qn ? qn + lane : src), wk = *(kn ? kn + lane : src);
    const float c = *(cos_t ? cos_t + (int64_t)s * 64 + lane : src);
    const float sn = *(cos_t ? sin_t + (int64_t)s * 64 + lane : src);
#pragma unroll
    for (int j = 0; j < 16; ++j) {
        if (j >= slots) continue;
        float x = xv[j];
        float *dst;
        if (j < H) {
            dst = q + (((int64_t)b * H + j) * S + s) * 64;
        } else if (j < H + nkv) {
            dst = k + (((int64_t)b * nkv + (j - H)) * S + s) * 64;
        } else {
            dst = v + (((int64_t)b * nkv + (j - H - nkv)) * S + s) * 64;
        }
        if (j < H + nkv) {
            const bool isq = j < H;
            if (isq ? qn != nullptr : kn != nullptr) {
                double ms = wave_sum_d((double)x * (double)x) / 64;
                const float sc = (float)(1.0 / sqrt(ms + 1e-6));
                x = x * sc * (isq ? wq : wk);
            }
            if (cos_t) {
                const float other = __shfl(x, lane < 32 ? lane + 32 : lane - 32, 64);
                x = lane < 32 ? x * c + (-other) * sn : x * c + other * sn;
            }
        }
        dst[lane] = x;
    }
}

// The additive mask of build_full_mask (ncp.c:361-386) for each of nb boards:
// prefix rows see only the prefix, target rows see the prefix and the
// target levels the pattern allows (block_diag: its own level; else levels
// at or below its own); prefix columns flagged in the board's pad flags (pad
// may be NULL) are -inf for every row (ncp.c:588-600).  lvl [T]: the level of
// each target row.
extern "C" __global__ void __launch_bounds__(256)
ncp_mask_k(float *__restrict__ mask, const int *__restrict__ lvl, const int *__restrict__ pad, int P, int T,
           int block_diag, int nb) {
    // nb boards: board b's mask at mask + b S S from its pad flags pad + b P
    const int S = P + T;
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (int64_t)nb * S * S) return;
    const int b = (int)(i / ((int64_t)S * S)), e = (int)(i - (int64_t)b * S * S);
    const int r = e / S, c = e % S;
    if (pad) pad += (int64_t)b * P;
    float v = 0.f;
    if (r < P && c >= P) {
        v = -INFINITY;
    } else if (r >= P && c >= P) {
        const int lr = lvl[r - P], lc = lvl[c - P];
        v = (block_diag ? lr == lc : lr >= lc) ? 0.f : -INFINITY;
    }
    if (pad && c < P && pad[c]) v = -INFINITY;
    mask[i] = v;
}

// h[(b S + off + t) C + c] = h[...] + tab[b tb + t C + c] for t < n (the
// level embedding added to the target rows, tb = 0; or a per-board table)
extern "C" __global__ void __launch_bounds__(256)
ncp_add_rows_k(float *__restrict__ h, const float *__restrict__ tab, int B, int S, int off, int n, int C,
               int64_t tb) {
#pragma clang fp contract(off)
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (int64_t)B * n * C) return;
    const int c = (int)(i % C);
    const int t = (int)((i / C) % n);
    const int b = (int)(i / ((int64_t)n * C));
    float *p = h + ((int64_t)b * S + off + t) * C + c;
    *p = *p + tab[(int64_t)b * tb + (int64_t)t * C + c];
}

// dst [B][n][C] = rows off .. off + n - 1 of each board of src [B][S][C]
extern "C" __global__ void __launch_bounds__(256)
ncp_gather_rows_k(const float *__restrict__ src, float *__restrict__ dst, int B, int S, int off, int n, int C) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (int64_t)B * n * C) return;
    const int c = (int)(i % C);
    const int64_t bt = i / C;
    const int t = (int)(bt % n), b = (int)(bt / n);
    dst[i] = src[((int64_t)b * S + off + t) * C + c];
}

// logits [B][T][maxV] rows off .. off + lk - 1 from lg [B][lk][V], -inf past V
// (ncp.c:601-637)
extern "C" __global__ void __launch_bounds__(256)
ncp_logits_k(const float *__restrict__ lg, float *__restrict__ logits, int B, int T, int off, int lk, int V,
             int maxV) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (int64_t)B * lk * maxV) return;
    const int v = (int)(i % maxV);
    const int64_t bt = i / maxV;
    const int t = (int)(bt % lk), b = (int)(bt / lk);
    logits[((int64_t)b * T + off + t) * maxV + v] = v < V ? lg[bt * V + v] : -INFINITY;
}

// |E_v|^2 in fp64, serial over d (ncp.c:448-451)
extern "C" __global__ void __launch_bounds__(256)
ncp_esq_k(const float *__restrict__ E, double *__restrict__ esq, int V, int Dd) {
#pragma clang fp contract(off)
    const int v = blockIdx.x * 256 + threadIdx.x;
    if (v >= V) return;
    const float *e = E + (int64_t)v * Dd;
    double s = 0;
    for (int d = 0; d < Dd; ++d) s += (double)e[d] * e[d];
    esq[v] = s;
}

// ds = (serial fp64 sum of esq over v) / V (ncp.c:452-453); one thread
extern "C" __global__ void ncp_dscale_k(const double *__restrict__ esq, double *__restrict__ ds, int V) {
#pragma clang fp contract(off)
    if (blockIdx.x != 0 || threadIdx.x != 0) return;
    double s = 0;
    for (int v = 0; v < V; ++v) s += esq[v];
    *ds = s / V;
}

// the codebook-tied head (ncp.c:454-466): out[r][v] = (float)((2 dot -
// esq[v]) / ds * invT (+ bias[v])), dot serial fp64 over d
extern "C" __global__ void __launch_bounds__(256)
ncp_tied_head_k(const float *__restrict__ z, const float *__restrict__ E, const double *__restrict__ esq,
                const double *__restrict__ ds, float invT, const float *__restrict__ bias, float *__restrict__ out,
                int rows, int V, int Dd) {
#pragma clang fp contract(off)
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (int64_t)rows * V) return;
    const int v = (int)(i % V);
    const int64_t r = i / V;
    const float *zr = z + r * Dd, *e = E + (int64_t)v * Dd;
    double dot = 0;
    for (int d = 0; d < Dd; ++d) dot += (double)zr[d] * e[d];
    double o = (2 * dot - esq[v]) / *ds * invT;
    if (bias) o += bias[v];
    out[i] = (float)o;
}
