// train.hip -- training-step kernels: LayerNorm/RMSNorm backward, softmax
// cross-entropy, AdamW, global-norm clipping and the SDPA backward.
//
// All gradients accumulate (+=) into the caller's buffers, as the tape
// backward of the reference does (train_tape.c:636-1051).
#include "ncm_dev.h"

// ---------------------------------------------------------------- norm backward
// One wave per row.  Row statistics in fp64 (train_tape.c:583-593 / 759-765)
// are written to stats[] for the parameter-gradient pass; dx follows the
// reference formulas in fp64 with one float rounding per element.
extern "C" __global__ void __launch_bounds__(256)
ln_bwd_rows(const float *__restrict__ x, const float *__restrict__ w, const float *__restrict__ dy,
            float *__restrict__ dx, double *__restrict__ stats, int64_t rows, int C, double eps) {
#pragma clang fp contract(off)
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= rows) return;
    const float *xr = x + row * C, *gr = dy + row * C;
    double mean = 0.0;
    for (int c = lane; c < C; c += 64) mean += (double)xr[c];
    mean = wave_sum_d(mean) / C;
    double var = 0.0;
    for (int c = lane; c < C; c += 64) {
        const double d = (double)xr[c] - mean;
        var += d * d;
    }
    var = wave_sum_d(var) / C;
    const double inv = 1.0 / sqrt(var + eps);
    if (lane == 0) {
        stats[2 * row] = mean;
        stats[2 * row + 1] = inv;
    }
    if (!dx) return;
    double dmean = 0.0, dvar = 0.0;
    for (int c = lane; c < C; c += 64) {
        const double d = (double)gr[c] * (w ? (double)w[c] : 1.0);
        dmean += d;
        dvar += d * ((double)xr[c] - mean);
    }
    dmean = wave_sum_d(dmean) / C;
    dvar = wave_sum_d(dvar) * (-0.5 * inv * inv * inv / C);
    float *dr = dx + row * C;
    for (int c = lane; c < C; c += 64) {
        const double d = (double)gr[c] * (w ? (double)w[c] : 1.0);
        dr[c] += (float)((d - dmean) * inv + 2 * ((double)xr[c] - mean) * dvar);
    }
}

extern "C" __global__ void __launch_bounds__(256)
rmsn_bwd_rows(const float *__restrict__ x, const float *__restrict__ w, const float *__restrict__ dy,
              float *__restrict__ dx, double *__restrict__ stats, int64_t rows, int C) {
#pragma clang fp contract(off)
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= rows) return;
    const float *xr = x + row * C, *gr = dy + row * C;
    double ms = 0.0;
    for (int c = lane; c < C; c += 64) ms += (double)xr[c] * (double)xr[c];
    ms = wave_sum_d(ms) / C;
    const double inv = 1.0 / sqrt(ms + 1e-6);
    if (lane == 0) stats[row] = inv;
    if (!dx) return;
    double dot = 0.0;
    for (int c = lane; c < C; c += 64) dot += (double)gr[c] * (w ? (double)w[c] : 1.0) * (double)xr[c];
    dot = wave_sum_d(dot) / C;
    float *dr = dx + row * C;
    for (int c = lane; c < C; c += 64) {
        const double wc = w ? (double)w[c] : 1.0;
        dr[c] += (float)(((double)gr[c] * wc - dot * (double)xr[c] * inv * inv) * inv);
    }
}

// Parameter gradients: per column, partial fp64 sums over a chunk of
// NORM_ROWS rows (ascending), then norm_param_final adds the chunk partials
// in chunk order and float-adds the rounded sum into dw / db.
//   kind 0 (LayerNorm): dw += sum dy*(x-mean)*inv, db += sum dy
//   kind 1 (RMSNorm):   dw += sum (float)(dy*x) * inv
#define NORM_ROWS 128
extern "C" __global__ void __launch_bounds__(256)
norm_param_partial(const float *__restrict__ x, const float *__restrict__ dy, const double *__restrict__ stats,
                   double *__restrict__ part, int64_t rows, int C, int kind) {
#pragma clang fp contract(off)
    const int c = blockIdx.x * 256 + threadIdx.x;
    if (c >= C) return;
    const int64_t r0 = (int64_t)blockIdx.y * NORM_ROWS;
    const int64_t r1 = r0 + NORM_ROWS < rows ? r0 + NORM_ROWS : rows;
    double sw = 0.0, sb = 0.0;
    for (int64_t r = r0; r < r1; ++r) {
        const float g = dy[r * C + c], xv = x[r * C + c];
        if (kind == 0) {
            sw += (double)g * (((double)xv - stats[2 * r]) * stats[2 * r + 1]);
            sb += (double)g;
        } else {
            const float gx = g * xv;
            sw += (double)gx * stats[r];
        }
    }
    double *p = part + ((int64_t)blockIdx.y * C + c) * 2;
    p[0] = sw;
    p[1] = sb;
}

extern "C" __global__ void __launch_bounds__(256)
norm_param_final(const double *__restrict__ part, float *__restrict__ dw, float *__restrict__ db, int chunks,
                 int C) {
    const int c = blockIdx.x * 256 + threadIdx.x;
    if (c >= C) return;
    double sw = 0.0, sb = 0.0;
    for (int k = 0; k < chunks; ++k) {
        sw += part[((int64_t)k * C + c) * 2];
        sb += part[((int64_t)k * C + c) * 2 + 1];
    }
    if (dw) dw[c] += (float)sw;
    if (db) db[c] += (float)sb;
}

// Fused norm backward for C <= 256 * NPL, C % 4 == 0 and 16-byte aligned rows:
// a workgroup owns NBF_ROWS consecutive rows, NBF_ROWS / 4 per wave in
// ascending order.  A row is read once into registers (float4 column group
// q = lane + 64 j of each operand) and the next row's loads are in flight
// while it is reduced: the row statistics, dx (the arithmetic of ln_bwd_rows /
// rmsn_bwd_rows) and the column partials of the parameter gradients (that of
// norm_param_partial) all come from those registers.  The four waves' column
// partials are added in wave order into part[chunk][C][2]; norm_param_sum adds
// the chunks in order.  x and dy are read once instead of twice and the row
// loop keeps its loads in flight instead of one scalar load per pass.
#define NBF_ROWS 32
// A row's float4 groups: every load unconditional (a column past C reads the
// row's last group and counts zero), so that a wave's loads of the next row
// stay in flight: a guarded load is a branch with a full wait at the join.
template <int KIND, int NPL>
__device__ __forceinline__ void nbf_load(const float *__restrict__ p, int64_t row, int C, int lane, f4 (&v)[NPL]) {
#pragma unroll
    for (int j = 0; j < NPL; ++j) {
        const int c = 4 * (lane + 64 * j);
        const f4 t = *(const f4 *)(p + row * C + min(c, C - 4));
        v[j] = c < C ? t : f4{0.f, 0.f, 0.f, 0.f};
    }
}

// MODE 0: dx = 0.0f + the gradient (a first write); 1: dx += the gradient;
// 2: dx = (0.0f + base) + the gradient, the bits of a first write of base
// followed by the accumulation (base: a residual gradient passed through)
template <int KIND, int NPL, int MODE>
__device__ __forceinline__ void norm_bwd_fused_body(const float *__restrict__ x, const float *__restrict__ w,
                                                    const float *__restrict__ dy, float *__restrict__ dx,
                                                    double *__restrict__ part, int64_t rows, int C, double eps,
                                                    const float *__restrict__ base) {
#pragma clang fp contract(off)
    constexpr int NP = KIND == 0 ? 2 : 1;   // parameter gradients: (dw, db) or dw
    __shared__ double red[3][64 * NPL][4][NP];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int64_t rbeg = (int64_t)blockIdx.x * NBF_ROWS + wave * (NBF_ROWS / 4);
    const int64_t rend = min(rows, rbeg + NBF_ROWS / 4);
    f4 wv[NPL];
    if (w) nbf_load<KIND, NPL>(w, 0, C, lane, wv);
#pragma unroll
    for (int j = 0; j < NPL; ++j)
        if (!w) wv[j] = f4{1.f, 1.f, 1.f, 1.f};
    double sp[NPL][4][NP];
#pragma unroll
    for (int j = 0; j < NPL; ++j)
#pragma unroll
        for (int e = 0; e < 4; ++e)
#pragma unroll
            for (int k = 0; k < NP; ++k) sp[j][e][k] = 0.0;
    f4 xa[NPL], ga[NPL];
    const int64_t r0 = min(rbeg, rows - 1);   // a wave past the last row loads a valid row and skips the loop
    nbf_load<KIND, NPL>(x, r0, C, lane, xa);
    nbf_load<KIND, NPL>(dy, r0, C, lane, ga);
    f4 ba[NPL];   // MODE 2: the base rows, loaded with x and dy one row ahead
    if constexpr (MODE == 2) nbf_load<KIND, NPL>(base, r0, C, lane, ba);
    for (int64_t r = rbeg; r < rend; ++r) {
        // the next row's loads (the last row again at the end), unconditionally
        f4 xn[NPL], gn[NPL];
        const int64_t rn = r + 1 < rend ? r + 1 : r;
        nbf_load<KIND, NPL>(x, rn, C, lane, xn);
        nbf_load<KIND, NPL>(dy, rn, C, lane, gn);
        f4 bn[NPL];
        if constexpr (MODE == 2) nbf_load<KIND, NPL>(base, rn, C, lane, bn);
        if (KIND == 0) {
            double mean = 0.0;
#pragma unroll
            for (int j = 0; j < NPL; ++j)
#pragma unroll
                for (int e = 0; e < 4; ++e) mean += (double)xa[j][e];
            mean = wave_sum_d(mean) / C;
            double var = 0.0;
#pragma unroll
            for (int j = 0; j < NPL; ++j)
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    if (4 * (lane + 64 * j) < C) {
                        const double d = (double)xa[j][e] - mean;
                        var += d * d;
                    }
            var = wave_sum_d(var) / C;
            const double inv = 1.0 / sqrt(var + eps);
            if (dx) {
                double dmean = 0.0, dvar = 0.0;
#pragma unroll
                for (int j = 0; j < NPL; ++j)
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        if (4 * (lane + 64 * j) < C) {
                            const double d = (double)ga[j][e] * (double)wv[j][e];
                            dmean += d;
                            dvar += d * ((double)xa[j][e] - mean);
                        }
                dmean = wave_sum_d(dmean) / C;
                dvar = wave_sum_d(dvar) * (-0.5 * inv * inv * inv / C);
#pragma unroll
                for (int j = 0; j < NPL; ++j) {
                    const int c = 4 * (lane + 64 * j);
                    if (c < C) {
                        f4 *o = (f4 *)(dx + r * C + c);
                        f4 v = f4{0.f, 0.f, 0.f, 0.f};
                        if constexpr (MODE == 1) v = *o;
                        if constexpr (MODE == 2) {
                            v = f4{0.0f + ba[j].x, 0.0f + ba[j].y, 0.0f + ba[j].z, 0.0f + ba[j].w};
                        }
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            const double d = (double)ga[j][e] * (double)wv[j][e];
                            v[e] += (float)((d - dmean) * inv + 2 * ((double)xa[j][e] - mean) * dvar);
                        }
                        *o = v;
                    }
                }
            }
#pragma unroll
            for (int j = 0; j < NPL; ++j)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    sp[j][e][0] += (double)ga[j][e] * (((double)xa[j][e] - mean) * inv);
                    sp[j][e][NP - 1] += (double)ga[j][e];
                }
        } else {
            double ms = 0.0;
#pragma unroll
            for (int j = 0; j < NPL; ++j)
#pragma unroll
                for (int e = 0; e < 4; ++e) ms += (double)xa[j][e] * (double)xa[j][e];
            ms = wave_sum_d(ms) / C;
            const double inv = 1.0 / sqrt(ms + 1e-6);
            if (dx) {
                double dot = 0.0;
#pragma unroll
                for (int j = 0; j < NPL; ++j)
#pragma unroll
                    for (int e = 0; e < 4; ++e) dot += (double)ga[j][e] * (double)wv[j][e] * (double)xa[j][e];
                dot = wave_sum_d(dot) / C;
#pragma unroll
                for (int j = 0; j < NPL; ++j) {
                    const int c = 4 * (lane + 64 * j);
                    if (c < C) {
                        f4 *o = (f4 *)(dx + r * C + c);
                        f4 v = f4{0.f, 0.f, 0.f, 0.f};
                        if constexpr (MODE == 1) v = *o;
                        if constexpr (MODE == 2) {
                            v = f4{0.0f + ba[j].x, 0.0f + ba[j].y, 0.0f + ba[j].z, 0.0f + ba[j].w};
                        }
#pragma unroll
                        for (int e = 0; e < 4; ++e)
                            v[e] += (float)(((double)ga[j][e] * (double)wv[j][e] -
                                             dot * (double)xa[j][e] * inv * inv) * inv);
                        *o = v;
                    }
                }
            }
#pragma unroll
            for (int j = 0; j < NPL; ++j)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float gx = ga[j][e] * xa[j][e];
                    sp[j][e][0] += (double)gx * inv;
                }
        }
#pragma unroll
        for (int j = 0; j < NPL; ++j) {
            xa[j] = xn[j];
            ga[j] = gn[j];
            if constexpr (MODE == 2) ba[j] = bn[j];
        }
    }
    if (!part) return;
    if (wave > 0) {
#pragma unroll
        for (int j = 0; j < NPL; ++j)
#pragma unroll
            for (int e = 0; e < 4; ++e)
#pragma unroll
                for (int k = 0; k < NP; ++k) red[wave - 1][lane + 64 * j][e][k] = sp[j][e][k];
    }
    __syncthreads();
    if (wave == 0) {
#pragma unroll
        for (int j = 0; j < NPL; ++j) {
            const int c = 4 * (lane + 64 * j);
            if (c >= C) continue;
            double *o = part + ((int64_t)blockIdx.x * C + c) * 2;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                double s0 = sp[j][e][0], s1 = sp[j][e][NP - 1];
#pragma unroll
                for (int v = 0; v < 3; ++v) {
                    s0 += red[v][lane + 64 * j][e][0];
                    s1 += red[v][lane + 64 * j][e][NP - 1];
                }
                o[2 * e] = s0;
                o[2 * e + 1] = KIND == 0 ? s1 : 0.0;
            }
        }
    }
}

#define NORM_BWD_FUSED(name, KIND, NPL)                                                                      \
    extern "C" __global__ void __launch_bounds__(256)                                                       \
        name(const float *__restrict__ x, const float *__restrict__ w, const float *__restrict__ dy,        \
             float *__restrict__ dx, double *__restrict__ part, int64_t rows, int C, double eps, int beta,    \
             const float *__restrict__ base) {                                                              \
        if (base)                                                                                           \
            norm_bwd_fused_body<KIND, NPL, 2>(x, w, dy, dx, part, rows, C, eps, base);                      \
        else if (beta)                                                                                      \
            norm_bwd_fused_body<KIND, NPL, 1>(x, w, dy, dx, part, rows, C, eps, base);                      \
        else                                                                                                \
            norm_bwd_fused_body<KIND, NPL, 0>(x, w, dy, dx, part, rows, C, eps, base);                      \
    }
NORM_BWD_FUSED(ln_bwd_fused_1, 0, 1)
NORM_BWD_FUSED(ln_bwd_fused_2, 0, 2)
NORM_BWD_FUSED(ln_bwd_fused_3, 0, 3)
NORM_BWD_FUSED(ln_bwd_fused_4, 0, 4)
NORM_BWD_FUSED(rmsn_bwd_fused_1, 1, 1)
NORM_BWD_FUSED(rmsn_bwd_fused_2, 1, 2)
NORM_BWD_FUSED(rmsn_bwd_fused_3, 1, 3)
NORM_BWD_FUSED(rmsn_bwd_fused_4, 1, 4)

// dw[c] += (float) sum_k part[k][c][0], db[c] += (float) sum_k part[k][c][1],
// the chunks added in order: a workgroup of 16 waves per 64 columns, wave v
// sums chunks v, v + 16, ... (32 loads in flight per batch), then wave 0 adds
// the 16 wave sums in wave order.
extern "C" __global__ void __launch_bounds__(1024)
norm_param_sum(const double *__restrict__ part, float *__restrict__ dw, float *__restrict__ db, int chunks, int C) {
    __shared__ double red[16][64][2];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int c = blockIdx.x * 64 + lane;
    double s0 = 0.0, s1 = 0.0;
    if (c < C) {
        const double *p = part + (int64_t)c * 2;
        for (int k0 = wave; k0 < chunks; k0 += 16 * 16) {
            double2 v[16];
#pragma unroll
            for (int u = 0; u < 16; ++u) {
                const int k = min(k0 + 16 * u, chunks - 1);
                v[u] = *(const double2 *)(p + (int64_t)k * C * 2);
            }
#pragma unroll
            for (int u = 0; u < 16; ++u)
                if (k0 + 16 * u < chunks) {
                    s0 += v[u].x;
                    s1 += v[u].y;
                }
        }
    }
    red[wave][lane][0] = s0;
    red[wave][lane][1] = s1;
    __syncthreads();
    if (wave == 0 && c < C) {
        double t0 = red[0][lane][0], t1 = red[0][lane][1];
#pragma unroll
        for (int v = 1; v < 16; ++v) {
            t0 += red[v][lane][0];
            t1 += red[v][lane][1];
        }
        if (dw) dw[c] += (float)t0;
        if (db) db[c] += (float)t1;
    }
}

// ---------------------------------------------------------------- cross-entropy
// One wave per row (train_tape.c:452-465): float max, fp64 exp and sum,
// p = (float)e / (float)den, nll = w * -log(p[tgt] + 1e-30).
//   mode 0: write probs
//   mode 1: dl += (float)((p - onehot) * w * inv), inv = weight / cnt with cnt
//           = cnt_in[0] when given, else cnt_val (fused forward + backward;
//           probs not stored)
// rowstat[2r] = nll contribution, rowstat[2r+1] = weight (0 for w == 0 rows).
// A target outside [0, V) (out-of-bounds in the reference) matches no class
// and contributes w * -log(1e-30).
extern "C" __global__ void __launch_bounds__(256)
ce_rows(const float *__restrict__ logits, const int *__restrict__ tgt, const float *__restrict__ wm,
        float *__restrict__ out, double *__restrict__ rowstat, const double *__restrict__ cnt_in,
        double cnt_val, double weight, int64_t rows, int V, int mode) {
#pragma clang fp contract(off)
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= rows) return;
    const float *l = logits + row * V;
    float m = -INFINITY;
    for (int v = lane; v < V; v += 64) m = fmaxf(m, l[v]);
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
    if (l[0] != l[0]) m = l[0];   // the reference's scan keeps a NaN first element
    double den = 0.0;
    for (int v = lane; v < V; v += 64) den += exp((double)l[v] - (double)m);
    den = wave_sum_d(den);
    const float fden = (float)den;
    const int t = tgt[row];
    const float w = wm ? wm[row] : 1.0f;
    if (mode == 0) {
        float *p = out + row * V;
        for (int v = lane; v < V; v += 64) p[v] = (float)exp((double)l[v] - (double)m) / fden;
    } else if (w != 0.0f) {
        const double cnt = cnt_in ? cnt_in[0] : cnt_val;
        const double inv = (cnt > 0 ? 1.0 / cnt : 0.0) * weight;
        float *g = out + row * V;
        for (int v = lane; v < V; v += 64) {
            const float p = (float)exp((double)l[v] - (double)m) / fden;
            g[v] += (float)(((double)p - (v == t ? 1.0 : 0.0)) * (double)w * inv);
        }
    }
    if (lane == 0) {
        double nll = 0.0, cw = 0.0;
        if (w != 0.0f) {
            const float pt = (unsigned)t < (unsigned)V ? (float)exp((double)l[t] - (double)m) / fden : 0.0f;
            nll = (double)w * -log((double)pt + 1e-30);
            cw = (double)w;
        }
        rowstat[2 * row] = nll;
        rowstat[2 * row + 1] = cw;
    }
}

// Weight count sum_r w_r (rows with w == 0 add nothing) for the fused mode.
extern "C" __global__ void __launch_bounds__(256)
ce_count(const float *__restrict__ wm, double *__restrict__ cnt, int64_t rows) {
    __shared__ double part[4];
    double s = 0.0;
    for (int64_t r = threadIdx.x; r < rows; r += 256) s += (double)wm[r];
    s = wave_sum_d(s);
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = s;
    __syncthreads();
    if (threadIdx.x == 0) cnt[0] = ((part[0] + part[1]) + part[2]) + part[3];
}

// loss = (float)(sum nll / sum w) over rowstat, fixed order (one workgroup).
extern "C" __global__ void __launch_bounds__(256)
ce_loss_final(const double *__restrict__ rowstat, float *__restrict__ loss, int64_t rows) {
    __shared__ double pn[4], pc[4];
    double n = 0.0, c = 0.0;
    for (int64_t r = threadIdx.x; r < rows; r += 256) {
        n += rowstat[2 * r];
        c += rowstat[2 * r + 1];
    }
    n = wave_sum_d(n);
    c = wave_sum_d(c);
    if ((threadIdx.x & 63) == 0) {
        pn[threadIdx.x >> 6] = n;
        pc[threadIdx.x >> 6] = c;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        const double nt = ((pn[0] + pn[1]) + pn[2]) + pn[3];
        const double ct = ((pc[0] + pc[1]) + pc[2]) + pc[3];
        loss[0] = ct > 0 ? (float)(nt / ct) : 0.0f;
    }
}

// k_ce_bwd (train_tape.c:1801-1810): dl += (float)((p - onehot) * w * inv).
extern "C" __global__ void __launch_bounds__(256)
ce_bwd_k(const float *__restrict__ probs, const int *__restrict__ tgt, const float *__restrict__ wm,
         float *__restrict__ dl, int64_t rows, int V, double inv) {
#pragma clang fp contract(off)
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= rows * V) return;
    const int64_t r = i / V;
    const int v = (int)(i - r * V);
    const float w = wm ? wm[r] : 1.0f;
    if (w == 0.0f) return;
    dl[i] += (float)(((double)probs[i] - (v == tgt[r] ? 1.0 : 0.0)) * (double)w * inv);
}

// ---------------------------------------------------------------- optimizer
// k_adamw (train.c:51-64), operation for operation: decoupled decay, moments
// in fp64 rounded to float, bias-corrected step in fp64.  Bit-identical to
// the host loop (train.c:131-141): IEEE double ops with contraction off.
extern "C" __global__ void __launch_bounds__(256)
adamw_k(float *__restrict__ p, float *__restrict__ g, float *__restrict__ m, float *__restrict__ v,
        int64_t n, double lr, double b1, double b2, double b1t, double b2t, double eps, double wd, int clear_g) {
#pragma clang fp contract(off)
    const int64_t k = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (k >= n) return;
    const float gk = g[k];
    if (clear_g) g[k] = 0.0f;   // the gradient, consumed, starts the next step at zero
    float pk = p[k];
    pk = pk - (float)(lr * wd * (double)pk);
    const float mk = (float)(b1 * (double)m[k] + (1.0 - b1) * (double)gk);
    const float vk = (float)(b2 * (double)v[k] + (1.0 - b2) * (double)gk * (double)gk);
    m[k] = mk;
    v[k] = vk;
    const double mh = (double)mk / b1t, vh = (double)vk / b2t;
    p[k] = pk - (float)(lr * mh / (sqrt(vh) + eps));
}

// Sum of squares in fp64: one partial per workgroup (grid-stride), written
// to part[blockIdx.x]; sumsq_final adds `count` partials in index order.
extern "C" __global__ void __launch_bounds__(256)
sumsq_partial(const float *__restrict__ g, int64_t n, double *__restrict__ part) {
    __shared__ double ws[4];
    double s = 0.0;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
        const double x = (double)g[i];
        s += x * x;
    }
    s = wave_sum_d(s);
    if ((threadIdx.x & 63) == 0) ws[threadIdx.x >> 6] = s;
    __syncthreads();
    if (threadIdx.x == 0) part[blockIdx.x] = ((ws[0] + ws[1]) + ws[2]) + ws[3];
}

extern "C" __global__ void __launch_bounds__(64)
sumsq_final(const double *__restrict__ part, int count, double *__restrict__ out) {
    double s = 0.0;
    for (int i = threadIdx.x; i < count; i += 64) s += part[i];
    s = wave_sum_d(s);
    if (threadIdx.x == 0) out[0] = s;
}

// ---- multi-tensor forms (one launch over a list of tensors) ----
// A tensor of the list: parameter, gradient, moments, size, learning-rate
// multiplier.  Must match struct MtTensor in train.c.
struct MtTensor {
    float *p, *g, *m, *v;
    int64_t n;
    double lr_mul;
};

// sumsq_partial over every tensor of the list in one launch, with the same
// partials: tensor i owns blocks [boff[i], boff[i+1]) (min(ceil(n/256), 1024)
// of them), and its block j sums elements j*256 + t, stepping by its own
// block count * 256, as sumsq_partial does with that grid.  The block's tensor
// is found by a binary search over boff staged in LDS (count <= MT_MAX).
#define MT_MAX 2048
extern "C" __global__ void __launch_bounds__(256)
sumsq_multi(const MtTensor *__restrict__ tt, const int *__restrict__ boff, int count, double *__restrict__ part) {
    __shared__ int so[MT_MAX + 1];
    __shared__ double ws[4];
    for (int i = threadIdx.x; i <= count; i += 256) so[i] = boff[i];
    __syncthreads();
    const int b = blockIdx.x;
    int lo = 0, hi = count - 1;   // last i with so[i] <= b
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (so[mid] <= b) lo = mid;
        else hi = mid - 1;
    }
    const int64_t nb = so[lo + 1] - so[lo], j = b - so[lo], n = tt[lo].n;
    const float *g = tt[lo].g;
    const int64_t st = nb * 256;
    double s = 0.0;
    // four loads in flight per pass (clamped index), added in element order
    for (int64_t i0 = j * 256 + threadIdx.x; i0 < n; i0 += 4 * st) {
        float x[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) x[u] = g[min(i0 + u * st, n - 1)];
#pragma unroll
        for (int u = 0; u < 4; ++u)
            if (i0 + u * st < n) s += (double)x[u] * (double)x[u];
    }
    s = wave_sum_d(s);
    if ((threadIdx.x & 63) == 0) ws[threadIdx.x >> 6] = s;
    __syncthreads();
    if (threadIdx.x == 0) part[b] = ((ws[0] + ws[1]) + ws[2]) + ws[3];
}

// sumsq_final, then the clip decision on the device: out[0] = sum of
// squares, scale[0] = (float)(1 / norm) when norm > max_norm, else 1 (a
// multiplication by 1.0f leaves every float as it is).
extern "C" __global__ void __launch_bounds__(64)
clip_final(const double *__restrict__ part, int count, double *__restrict__ out, float *__restrict__ scale,
           double max_norm) {
    double s = 0.0;
    // lane l adds partials l, l + 64, ... in order, 16 loads in flight per pass
    for (int i0 = threadIdx.x; i0 < count; i0 += 64 * 16) {
        double x[16];
#pragma unroll
        for (int u = 0; u < 16; ++u) x[u] = part[min(i0 + 64 * u, count - 1)];
#pragma unroll
        for (int u = 0; u < 16; ++u)
            if (i0 + 64 * u < count) s += x[u];
    }
    s = wave_sum_d(s);
    if (threadIdx.x == 0) {
        out[0] = s;
        const double gn = sqrt(s);
        scale[0] = gn > max_norm ? (float)(1.0 / gn) : 1.0f;
    }
}

// adamw_k over every tensor of the list in one launch: block b updates
// elements [start, start + len) of tensor ch[b].x (start = ch[b].y * len),
// reading the gradient times *scale (the in-place clip of the gradient
// followed by adamw_k, without writing the scaled gradient back) and, with
// clear_g, leaving the gradient zero.  lr of tensor i = lr * lr_mul.
extern "C" __global__ void __launch_bounds__(256)
adamw_multi(const MtTensor *__restrict__ tt, const int2 *__restrict__ ch, int len, const float *__restrict__ scale,
            double lr0, double b1, double b2, double b1t, double b2t, double eps, double wd, int clear_g) {
#pragma clang fp contract(off)
    const int2 c = ch[blockIdx.x];
    const MtTensor t = tt[c.x];
    const int64_t start = (int64_t)c.y * len, end = min(t.n, start + len);
    const float s = *scale;
    const double lr = lr0 * t.lr_mul;
    // four elements per pass, their loads issued together (clamped index)
    for (int64_t k0 = start + threadIdx.x; k0 < end; k0 += 1024) {
        float g4[4], p4[4], m4[4], v4[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int64_t k = min(k0 + 256 * u, end - 1);
            g4[u] = t.g[k];
            p4[u] = t.p[k];
            m4[u] = t.m[k];
            v4[u] = t.v[k];
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int64_t k = k0 + 256 * u;
            if (k >= end) continue;
            const float gk = g4[u] * s;
            if (clear_g) t.g[k] = 0.0f;
            float pk = p4[u];
            pk = pk - (float)(lr * wd * (double)pk);
            const float mk = (float)(b1 * (double)m4[u] + (1.0 - b1) * (double)gk);
            const float vk = (float)(b2 * (double)v4[u] + (1.0 - b2) * (double)gk * (double)gk);
            t.m[k] = mk;
            t.v[k] = vk;
            const double mh = (double)mk / b1t, vh = (double)vk / b2t;
            t.p[k] = pk - (float)(lr * mh / (sqrt(vh) + eps));
        }
    }
}

extern "C" __global__ void __launch_bounds__(256)
scale_inplace_k(float *__restrict__ g, int64_t n, float s) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i < n) g[i] = g[i] * s;
}

// ---------------------------------------------------------------- SDPA backward
// Inputs: q [B][H][Tq][hd], k/v [B][Hkv][Tkv][hd], the stored probabilities
// P [B][H][Tq][Tkv] (train_tape.c:289-313), dO like q.  With dP = dO V^T and
// D = rowsum(P o dP):  dS = P o (dP - D),  dq += scale dS K,
// dk += scale dS^T Q,  dv += P^T dO (kv head = h / (H/Hkv); dk, dv sum over
// the query heads of the group) -- train_tape.c:936-1051.
//
// Generic path (any hd <= 256, any Tkv): one wave per row, lanes over d.
// sdpa_bwd_dq_rows also writes D for sdpa_bwd_dkdv_rows.
extern "C" __global__ void __launch_bounds__(256)
sdpa_bwd_dq_rows(const float *__restrict__ k, const float *__restrict__ v, const float *__restrict__ P,
                 const float *__restrict__ dO, float *__restrict__ dq, float *__restrict__ Dout, int B, int H,
                 int Hkv, int Tq, int Tkv, int hd, float scale) {
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= (int64_t)B * H * Tq) return;
    const int h = (int)((row / Tq) % H), b = (int)(row / ((int64_t)Tq * H));
    const int kvh = h / (H / Hkv);
    const float *kb = k + ((int64_t)b * Hkv + kvh) * Tkv * hd;
    const float *vb = v + ((int64_t)b * Hkv + kvh) * Tkv * hd;
    const float *pr = P + row * Tkv;
    float g[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int d = lane + 64 * j;
        g[j] = d < hd ? dO[row * hd + d] : 0.f;
    }
    double tot = 0.0;
    for (int tk = 0; tk < Tkv; ++tk) {
        const float *vr = vb + (int64_t)tk * hd;
        double s = 0.0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int d = lane + 64 * j;
            if (d < hd) s += (double)g[j] * (double)vr[d];
        }
        tot += wave_sum_d(s) * (double)pr[tk];
    }
    if (lane == 0 && Dout) Dout[row] = (float)tot;
    if (!dq) return;
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
    for (int tk = 0; tk < Tkv; ++tk) {
        const float *vr = vb + (int64_t)tk * hd, *kr = kb + (int64_t)tk * hd;
        double s = 0.0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int d = lane + 64 * j;
            if (d < hd) s += (double)g[j] * (double)vr[d];
        }
        const double p = (double)pr[tk];
        const float ds = (float)(p * wave_sum_d(s) - p * tot);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int d = lane + 64 * j;
            if (d < hd) acc[j] += ds * kr[d];
        }
    }
    float *o = dq + row * hd;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int d = lane + 64 * j;
        if (d < hd) o[d] += scale * acc[j];
    }
}

// One wave per (b, kv head, key): lanes over d; sums over the query heads of
// the group and all queries.
extern "C" __global__ void __launch_bounds__(256)
sdpa_bwd_dkdv_rows(const float *__restrict__ q, const float *__restrict__ v, const float *__restrict__ P,
                   const float *__restrict__ dO, const float *__restrict__ D, float *__restrict__ dk,
                   float *__restrict__ dv, int B, int H, int Hkv, int Tq, int Tkv, int hd, float scale) {
    const int64_t kr_ = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (kr_ >= (int64_t)B * Hkv * Tkv) return;
    const int tk = (int)(kr_ % Tkv);
    const int kvh = (int)((kr_ / Tkv) % Hkv), b = (int)(kr_ / ((int64_t)Tkv * Hkv));
    const int rep = H / Hkv;
    const float *vr = v + kr_ * hd;
    float vv[4], sk[4] = {0.f, 0.f, 0.f, 0.f}, sv[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int d = lane + 64 * j;
        vv[j] = d < hd ? vr[d] : 0.f;
    }
    for (int h = kvh * rep; h < (kvh + 1) * rep; ++h) {
        const int64_t rbase = ((int64_t)b * H + h) * Tq;
        for (int tq = 0; tq < Tq; ++tq) {
            const int64_t row = rbase + tq;
            const float *gr = dO + row * hd, *qr = q + row * hd;
            double s = 0.0;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int d = lane + 64 * j;
                if (d < hd) s += (double)gr[d] * (double)vv[j];
            }
            const double p = (double)P[row * Tkv + tk];
            const float ds = (float)(p * wave_sum_d(s) - p * (double)D[row]);
            const float pf = (float)p;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int d = lane + 64 * j;
                if (d < hd) {
                    sk[j] += ds * qr[d];
                    sv[j] += pf * gr[d];
                }
            }
        }
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int d = lane + 64 * j;
        if (d < hd) {
            if (dk) dk[kr_ * hd + d] += scale * sk[j];
            if (dv) dv[kr_ * hd + d] += sv[j];
        }
    }
}

// MFMA path for hd = 64 (Tkv % 4 == 0, 16-byte aligned pointers).
// k-permutation as in the GEMM: MFMA step s gives lane group g the reduction
// index 4g + s, so every operand fragment is a float4.
#define SB_LD 72

// dq kernel: a workgroup owns 64 queries of one (b, h), wave w the 16
// queries q0 + 16w + li.  Sweep 1 builds D = sum_k P dP; sweep 2 forms
// dS^T = P^T o (dP^T - D) in the accumulator layout of dP^T = V dO^T (lane
// (li, g) holds keys 16c + 4g + r of query li), which is the A operand of
// dq = dS K.
extern "C" __global__ void __launch_bounds__(256)
sdpa_bwd_dq_hd64(const float *__restrict__ k, const float *__restrict__ v, const float *__restrict__ P,
                 const float *__restrict__ dO, float *__restrict__ dq, float *__restrict__ Dout, int H, int Hkv,
                 int Tq, int Tkv, float scale) {
    __shared__ __attribute__((aligned(16))) float sK[64 * SB_LD];
    __shared__ __attribute__((aligned(16))) float sV[64 * SB_LD];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int li = lane & 15, lg = lane >> 4;
    const int h = blockIdx.y, b = blockIdx.z;
    const int kvh = h / (H / Hkv);
    const int qw = blockIdx.x * 64 + wave * 16;
    const int my_q = qw + li;
    const int64_t rbase = ((int64_t)b * H + h) * Tq;
    const float *kb = k + ((int64_t)b * Hkv + kvh) * Tkv * 64;
    const float *vb = v + ((int64_t)b * Hkv + kvh) * Tkv * 64;
    const float *prow = P + (rbase + (my_q < Tq ? my_q : 0)) * Tkv;

    f4 gf[4];   // dO^T fragments: query my_q, d = 16kc + 4g .. +3
#pragma unroll
    for (int kc = 0; kc < 4; ++kc)
        gf[kc] = my_q < Tq ? *(const f4 *)(dO + (rbase + my_q) * 64 + kc * 16 + 4 * lg) : f4{0.f, 0.f, 0.f, 0.f};

    float tot = 0.f;
    f4 acc[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) acc[u] = f4{0.f, 0.f, 0.f, 0.f};

    for (int sweep = 0; sweep < 2; ++sweep) {
        for (int k0 = 0; k0 < Tkv; k0 += 64) {
            __syncthreads();
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int f = tid + j * 256;
                const int r = f >> 4, c = (f & 15) * 4;
                const int key = k0 + r;
                f4 vv = {0.f, 0.f, 0.f, 0.f}, kv = {0.f, 0.f, 0.f, 0.f};
                if (key < Tkv) {
                    vv = *(const f4 *)(vb + (int64_t)key * 64 + c);
                    if (sweep) kv = *(const f4 *)(kb + (int64_t)key * 64 + c);
                }
                *(f4 *)(sV + r * SB_LD + LDS_SWZ(r, c)) = vv;
                if (sweep) *(f4 *)(sK + r * SB_LD + LDS_SWZ(r, c)) = kv;
            }
            __syncthreads();
            // dP^T[c]: keys k0 + 16c + 4g + r, query my_q
            f4 dp[4], pv[4];
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                dp[c] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int kc = 0; kc < 4; ++kc) {
                    const f4 vf = *(const f4 *)(sV + (16 * c + li) * SB_LD + LDS_SWZ((16 * c + li), kc * 16 + 4 * lg));
#pragma unroll
                    for (int st = 0; st < 4; ++st) dp[c] = mfma4(vf[st], gf[kc][st], dp[c]);
                }
                const int key = k0 + 16 * c + 4 * lg;
                pv[c] = (my_q < Tq && key < Tkv) ? *(const f4 *)(prow + key) : f4{0.f, 0.f, 0.f, 0.f};
            }
            if (sweep == 0) {
#pragma unroll
                for (int c = 0; c < 4; ++c)
#pragma unroll
                    for (int r = 0; r < 4; ++r) tot += pv[c][r] * dp[c][r];
            } else {
#pragma unroll
                for (int c = 0; c < 4; ++c)
#pragma unroll
                    for (int r = 0; r < 4; ++r) dp[c][r] = pv[c][r] * (dp[c][r] - tot);
                // dq[query qw + 4g + r][d = 4li + u] += dS[query][key] K[key][d]
#pragma unroll
                for (int c = 0; c < 4; ++c)
#pragma unroll
                    for (int st = 0; st < 4; ++st) {
                        const f4 kf = *(const f4 *)(sK + (16 * c + 4 * lg + st) * SB_LD + LDS_SWZ((16 * c + 4 * lg + st), 4 * li));
#pragma unroll
                        for (int u = 0; u < 4; ++u) acc[u] = mfma4(dp[c][st], kf[u], acc[u]);
                    }
            }
        }
        if (sweep == 0) {
            tot += __shfl_xor(tot, 16, 64);
            tot += __shfl_xor(tot, 32, 64);
            if (lg == 0 && my_q < Tq && Dout) Dout[rbase + my_q] = tot;
            if (!dq) return;
        }
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int qi = qw + 4 * lg + r;
        if (qi < Tq) {
            f4 *o = (f4 *)(dq + (rbase + qi) * 64 + 4 * li);
            f4 cur = *o;
            cur[0] += scale * acc[0][r];
            cur[1] += scale * acc[1][r];
            cur[2] += scale * acc[2][r];
            cur[3] += scale * acc[3][r];
            *o = cur;
        }
    }
}

// dk/dv kernel: a workgroup owns 64 keys of one (b, kv head), wave w the 16
// keys k0 + 16w + li.  For every query head of the group and every 64-query
// tile: dP = dO V^T in the layout (query 16c + 4g + r, key li) -- the A
// operand layout of dV = P^T dO and dK = dS^T Q.  P^T is staged in LDS with
// the float4 column groups XOR-swizzled by (key & 15), so both the
// transposing stores and the float4 loads are free of bank conflicts.
extern "C" __global__ void __launch_bounds__(256)
sdpa_bwd_dkdv_hd64(const float *__restrict__ q, const float *__restrict__ v, const float *__restrict__ P,
                   const float *__restrict__ dO, const float *__restrict__ D, float *__restrict__ dk,
                   float *__restrict__ dv, int H, int Hkv, int Tq, int Tkv, float scale) {
    __shared__ __attribute__((aligned(16))) float sG[64 * SB_LD];   // dO tile [query][d]
    __shared__ __attribute__((aligned(16))) float sQ[64 * SB_LD];   // Q tile  [query][d]
    __shared__ __attribute__((aligned(16))) float sPT[64 * 64];     // P^T     [key][query], swizzled
    __shared__ __attribute__((aligned(16))) float sD[64];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int li = lane & 15, lg = lane >> 4;
    const int kvh = blockIdx.y, b = blockIdx.z;
    const int rep = H / Hkv;
    const int k0 = blockIdx.x * 64;
    const int kl = wave * 16 + li;            // this lane's key within the tile
    const int my_k = k0 + kl;
    const int64_t kbase = ((int64_t)b * Hkv + kvh) * Tkv;

    f4 vf[4];   // V fragments: key my_k, d = 16kc + 4g .. +3
#pragma unroll
    for (int kc = 0; kc < 4; ++kc)
        vf[kc] = my_k < Tkv ? *(const f4 *)(v + (kbase + my_k) * 64 + kc * 16 + 4 * lg) : f4{0.f, 0.f, 0.f, 0.f};

    f4 ak[4], av[4];   // [u][r]: key k0 + 16w + 4g + r, d = 4li + u
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        ak[u] = f4{0.f, 0.f, 0.f, 0.f};
        av[u] = f4{0.f, 0.f, 0.f, 0.f};
    }

    for (int h = kvh * rep; h < (kvh + 1) * rep; ++h) {
        const int64_t rbase = ((int64_t)b * H + h) * Tq;
        for (int q0 = 0; q0 < Tq; q0 += 64) {
            __syncthreads();
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                // dO and Q rows: float4 along d
                const int f = tid + j * 256;
                const int r = f >> 4, c = (f & 15) * 4;
                const int qi = q0 + r;
                f4 gv = {0.f, 0.f, 0.f, 0.f}, qv = {0.f, 0.f, 0.f, 0.f};
                if (qi < Tq) {
                    gv = *(const f4 *)(dO + (rbase + qi) * 64 + c);
                    qv = *(const f4 *)(q + (rbase + qi) * 64 + c);
                }
                *(f4 *)(sG + r * SB_LD + LDS_SWZ(r, c)) = gv;
                *(f4 *)(sQ + r * SB_LD + LDS_SWZ(r, c)) = qv;
                // P rows (query r2, keys 4c2 .. +3) stored transposed
                const int r2 = f & 63, c2 = f >> 6;
                const int qj = q0 + r2, key = k0 + 4 * c2;
                f4 pv = {0.f, 0.f, 0.f, 0.f};
                if (qj < Tq && key < Tkv) pv = *(const f4 *)(P + (rbase + qj) * Tkv + key);
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int kk = 4 * c2 + e;
                    sPT[kk * 64 + ((((r2 >> 2) ^ (kk & 15))) << 2) + (r2 & 3)] = pv[e];
                }
            }
            if (tid < 64) sD[tid] = q0 + tid < Tq ? D[rbase + q0 + tid] : 0.f;
            __syncthreads();

            // dP[c] (query 16c + 4g + r, key kl), P in the same layout, dS
            f4 dp[4], pf[4];
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                dp[c] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int kc = 0; kc < 4; ++kc) {
                    const f4 gfr = *(const f4 *)(sG + (16 * c + li) * SB_LD + LDS_SWZ((16 * c + li), kc * 16 + 4 * lg));
#pragma unroll
                    for (int st = 0; st < 4; ++st) dp[c] = mfma4(gfr[st], vf[kc][st], dp[c]);
                }
                pf[c] = *(const f4 *)(sPT + kl * 64 + (((4 * c + lg) ^ (kl & 15)) << 2));
                const f4 dd = *(const f4 *)(sD + 16 * c + 4 * lg);
#pragma unroll
                for (int r = 0; r < 4; ++r) dp[c][r] = pf[c][r] * (dp[c][r] - dd[r]);
            }
            // dV += P^T dO, dK += dS^T Q
#pragma unroll
            for (int c = 0; c < 4; ++c)
#pragma unroll
                for (int st = 0; st < 4; ++st) {
                    const f4 gfr = *(const f4 *)(sG + (16 * c + 4 * lg + st) * SB_LD + LDS_SWZ((16 * c + 4 * lg + st), 4 * li));
                    const f4 qfr = *(const f4 *)(sQ + (16 * c + 4 * lg + st) * SB_LD + LDS_SWZ((16 * c + 4 * lg + st), 4 * li));
#pragma unroll
                    for (int u = 0; u < 4; ++u) {
                        av[u] = mfma4(pf[c][st], gfr[u], av[u]);
                        ak[u] = mfma4(dp[c][st], qfr[u], ak[u]);
                    }
                }
        }
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int key = k0 + wave * 16 + 4 * lg + r;
        if (key < Tkv) {
            if (dk) {
                f4 *o = (f4 *)(dk + (kbase + key) * 64 + 4 * li);
                f4 cur = *o;
                cur[0] += scale * ak[0][r];
                cur[1] += scale * ak[1][r];
                cur[2] += scale * ak[2][r];
                cur[3] += scale * ak[3][r];
                *o = cur;
            }
            if (dv) {
                f4 *o = (f4 *)(dv + (kbase + key) * 64 + 4 * li);
                f4 cur = *o;
                cur[0] += av[0][r];
                cur[1] += av[1][r];
                cur[2] += av[2][r];
                cur[3] += av[3][r];
                *o = cur;
            }
        }
    }
}

// ---------------------------------------------------------------- stored probabilities
// P = softmax(Q K^T * scale + mask) per row, written [B][H][Tq][Tkv]: the
// probabilities the tape keeps for the SDPA backward (train_tape.c:289-313
// builds them on the host).  sdpa_probs_hd64: 64 queries per workgroup,
// S^T = K Q^T on MFMA as in the forward; pass 1 finds the row max and sum,
// pass 2 writes exp(s - max) / sum.  Keys past Tkv are not written.
extern "C" __global__ void __launch_bounds__(256)
sdpa_probs_hd64(const float *__restrict__ q, const float *__restrict__ k, const float *__restrict__ mask,
                float *__restrict__ P, int H, int Hkv, int Tq, int Tkv, float scale) {
    __shared__ __attribute__((aligned(16))) float sK[64 * SB_LD];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int li = lane & 15, lg = lane >> 4;
    const int h = blockIdx.y, b = blockIdx.z;
    const int kvh = h / (H / Hkv);
    const int my_q = blockIdx.x * 64 + wave * 16 + li;
    const int64_t rbase = ((int64_t)b * H + h) * Tq;
    const float *kb = k + ((int64_t)b * Hkv + kvh) * Tkv * 64;
    f4 qf[4];
#pragma unroll
    for (int kc = 0; kc < 4; ++kc)
        qf[kc] = my_q < Tq ? *(const f4 *)(q + (rbase + my_q) * 64 + kc * 16 + 4 * lg) : f4{0.f, 0.f, 0.f, 0.f};
    float m_run = -INFINITY, l_run = 0.f, inv = 0.f;
    for (int pass = 0; pass < 2; ++pass) {
        for (int k0 = 0; k0 < Tkv; k0 += 64) {
            __syncthreads();
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int f = tid + j * 256;
                const int r = f >> 4, c = (f & 15) * 4;
                const int key = k0 + r;
                *(f4 *)(sK + r * SB_LD + LDS_SWZ(r, c)) = key < Tkv ? *(const f4 *)(kb + (int64_t)key * 64 + c)
                                                        : f4{0.f, 0.f, 0.f, 0.f};
            }
            __syncthreads();
            f4 s[4];
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                s[c] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int kc = 0; kc < 4; ++kc) {
                    const f4 kf = *(const f4 *)(sK + (16 * c + li) * SB_LD + LDS_SWZ((16 * c + li), kc * 16 + 4 * lg));
#pragma unroll
                    for (int st = 0; st < 4; ++st) s[c] = mfma4(kf[st], qf[kc][st], s[c]);
                }
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int key = k0 + 16 * c + 4 * lg + r;
                    float x = s[c][r] * scale;
                    if (mask && key < Tkv && my_q < Tq) x += mask[(int64_t)my_q * Tkv + key];
                    s[c][r] = key < Tkv ? x : -INFINITY;
                }
            }
            if (pass == 0) {
                float mt = -INFINITY;
#pragma unroll
                for (int c = 0; c < 4; ++c)
#pragma unroll
                    for (int r = 0; r < 4; ++r) mt = fmaxf(mt, s[c][r]);
                const float m_new = fmaxf(m_run, mt);
                float ps = 0.f;
                if (m_new != -INFINITY) {
#pragma unroll
                    for (int c = 0; c < 4; ++c)
#pragma unroll
                        for (int r = 0; r < 4; ++r) ps += __expf(s[c][r] - m_new);
                    l_run = l_run * __expf(m_run - m_new) + ps;
                    m_run = m_new;
                }
            } else if (my_q < Tq) {
                float *pr = P + (rbase + my_q) * Tkv;
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    const int key = k0 + 16 * c + 4 * lg;
                    f4 pv;
#pragma unroll
                    for (int r = 0; r < 4; ++r) pv[r] = __expf(s[c][r] - m_run) * inv;
                    if (key + 3 < Tkv) {
                        *(f4 *)(pr + key) = pv;
                    } else {
#pragma unroll
                        for (int r = 0; r < 4; ++r)
                            if (key + r < Tkv) pr[key + r] = pv[r];
                    }
                }
            }
        }
        if (pass == 0) {
            // combine the four lane groups' (max, sum) of query li
#pragma unroll
            for (int o = 16; o <= 32; o <<= 1) {
                const float mo = __shfl_xor(m_run, o, 64), lo = __shfl_xor(l_run, o, 64);
                const float mn = fmaxf(m_run, mo);
                if (mn != -INFINITY) {
                    l_run = l_run * __expf(m_run - mn) + lo * __expf(mo - mn);
                    m_run = mn;
                }
            }
            inv = 1.0f / l_run;
        }
    }
}

// Generic stored probabilities (any hd <= 256): one wave per query row.
extern "C" __global__ void __launch_bounds__(256)
sdpa_probs_rows(const float *__restrict__ q, const float *__restrict__ k, const float *__restrict__ mask,
                float *__restrict__ P, int B, int H, int Hkv, int Tq, int Tkv, int hd, float scale) {
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= (int64_t)B * H * Tq) return;
    const int tq = (int)(row % Tq);
    const int h = (int)((row / Tq) % H), b = (int)(row / ((int64_t)Tq * H));
    const int kvh = h / (H / Hkv);
    const float *kb = k + ((int64_t)b * Hkv + kvh) * Tkv * hd;
    float qv[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int d = lane + 64 * j;
        qv[j] = d < hd ? q[row * hd + d] : 0.f;
    }
    float *pr = P + row * Tkv;
    // pass 1: online max and sum; pass 2: recompute each score and write p
    float m = -INFINITY, l = 0.f;
    for (int pass = 0; pass < 2; ++pass) {
        for (int tk = 0; tk < Tkv; ++tk) {
            float dot = 0.f;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int d = lane + 64 * j;
                if (d < hd) dot += qv[j] * kb[(int64_t)tk * hd + d];
            }
            float x = wave_sum(dot) * scale;
            if (mask) x += mask[(int64_t)tq * Tkv + tk];
            if (pass == 0) {
                const float mn = fmaxf(m, x);
                if (mn != -INFINITY) {
                    l = l * __expf(m - mn) + __expf(x - mn);
                    m = mn;
                }
            } else if (lane == 0) {
                pr[tk] = __expf(x - m) / l;
            }
        }
    }
}

// ---------------------------------------------------------------- elementwise backward
// train_tape.c:830-873: dx += (float)(dy * g(x)), g in fp64.
// kind 0 gelu (erf), 1 silu, 2 gelu_tanh (gelu_new).
extern "C" __global__ void __launch_bounds__(256)
act_bwd_k(const float *__restrict__ x, const float *__restrict__ dy, float *__restrict__ dx, int64_t n, int kind) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    dx[i] += act_bwd_one(x[i], dy[i], kind);
}

// The same on float4 groups (n4 = n / 4, 16-byte aligned): four independent
// fp64 evaluations per thread.
extern "C" __global__ void __launch_bounds__(256)
act_bwd4_k(const float *__restrict__ x, const float *__restrict__ dy, float *__restrict__ dx, int64_t n4, int kind,
           int beta) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n4) return;
    const f4 xv = ((const f4 *)x)[i], g = ((const f4 *)dy)[i];
    f4 d = beta ? ((const f4 *)dx)[i] : f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int e = 0; e < 4; ++e) d[e] += act_bwd_one(xv[e], g[e], kind);
    ((f4 *)dx)[i] = d;
}

// train_tape.c:1254-1268: da += dy*b, db += dy*a (float products)
extern "C" __global__ void __launch_bounds__(256)
mul_bwd_k(const float *__restrict__ a, const float *__restrict__ b, const float *__restrict__ dy,
          float *__restrict__ da, float *__restrict__ db, int64_t n) {
#pragma clang fp contract(off)
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    const float g = dy[i];
    if (da) da[i] += g * b[i];
    if (db) db[i] += g * a[i];
}

// train_tape.c:890-930 (k_rope_bwd): transposed rotation in fp64; one thread
// per (row, d < hd/2), position row % T.
extern "C" __global__ void __launch_bounds__(256)
rope_bwd_k(float *__restrict__ dx, const float *__restrict__ g, const float *__restrict__ cos_t,
           const float *__restrict__ sin_t, int64_t rows, int T, int hd) {
#pragma clang fp contract(off)
    const int h = hd >> 1;
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= rows * h) return;
    const int64_t row = i / h;
    const int d = (int)(i - row * h);
    const int t = (int)(row % T);
    const float *gr = g + row * hd, *co = cos_t + (int64_t)t * hd, *si = sin_t + (int64_t)t * hd;
    const double g0 = gr[d], g1 = gr[d + h];
    const double c0 = co[d], s0 = si[d], c1 = co[d + h], s1 = si[d + h];
    dx[row * hd + d] += (float)(g0 * c0 + g1 * s1);
    dx[row * hd + h + d] += (float)(-g0 * s0 + g1 * c1);
}

// train_tape.c:726-741 TOP_EMBED: rows grouped by id on the host (ids in
// ascending row order, as the reference visits them); per (id, d) a float
// sum in that order, float-added into dW -- bit-identical to the reference.
extern "C" __global__ void __launch_bounds__(256)
emb_bwd_k(const float *__restrict__ dy, const int *__restrict__ uid, const int *__restrict__ off,
          const int *__restrict__ rowlist, float *__restrict__ dW, int D) {
#pragma clang fp contract(off)
    const int d = blockIdx.x * 256 + threadIdx.x;
    if (d >= D) return;
    const int u = blockIdx.y;
    float s = 0.f;
    for (int j = off[u]; j < off[u + 1]; ++j) s += dy[(int64_t)rowlist[j] * D + d];
    float *w = dW + (int64_t)uid[u] * D + d;
    *w = *w + s;
}

// train_tape.c:1293-1328 TOP_SPLIT: one thread per element of the fused
// input row [B][T][C + 2*K*hd]; k/v gradients summed over the query heads
// of the kv head (float, ascending h).
extern "C" __global__ void __launch_bounds__(256)
qkv_split_bwd_k(const float *__restrict__ gq, const float *__restrict__ gk, const float *__restrict__ gv,
                float *__restrict__ dx, int B, int T, int C, int H, int hd, int K, int rep) {
#pragma clang fp contract(off)
    const int64_t row_len = (int64_t)C + 2 * K * hd;
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (int64_t)B * T * row_len) return;
    const int64_t bt = i / row_len;
    const int col = (int)(i - bt * row_len);
    const int t = (int)(bt % T), b = (int)(bt / T);
    if (col < C) {
        if (!gq) return;
        const int h = col / hd, d = col - h * hd;
        if (h < H) dx[i] += gq[(((int64_t)b * H + h) * T + t) * hd + d];
        return;
    }
    const int kc = col - C;
    const float *g = kc < K * hd ? gk : gv;
    if (!g) return;
    const int kk = kc < K * hd ? kc : kc - K * hd;
    const int kvh = kk / hd, d = kk - kvh * hd;
    float s = 0.f;
    for (int h = kvh * rep; h < (kvh + 1) * rep && h < H; ++h) s += g[(((int64_t)b * H + h) * T + t) * hd + d];
    dx[i] += s;
}

// Row-blocked forms of qkv_split_bwd_k and heads_bwd_k (the same float
// operations per element) for hd and C multiples of 4 and 16-byte aligned
// operands: one workgroup per (b, t) row, one float4 per thread and pass,
// the row's indices computed once in 32-bit.
__device__ __forceinline__ void rows_bt(int T, int H, int hd, int &bt, int64_t &base, int64_t &hs) {
    bt = blockIdx.x;
    const int b = bt / T, t = bt - b * T;
    hs = (int64_t)T * hd;
    base = ((int64_t)b * H * T + t) * hd;
}

extern "C" __global__ void __launch_bounds__(256)
qkv_split_bwd_rows_k(const float *__restrict__ gq, const float *__restrict__ gk, const float *__restrict__ gv,
                     float *__restrict__ dx, int T, int C, int H, int hd, int K, int rep, int beta) {
#pragma clang fp contract(off)
    int bt;
    int64_t base, hs;
    rows_bt(T, H, hd, bt, base, hs);
    const int rl = C + 2 * K * hd;
    f4 *row = (f4 *)(dx + (int64_t)bt * rl);
    for (int f = threadIdx.x; f < rl / 4; f += 256) {
        const int c = 4 * f;
        const f4 z = {0.f, 0.f, 0.f, 0.f};
        if (c < C) {
            const int h = c / hd;
            if (gq && h < H) row[f] = (beta ? row[f] : z) + *(const f4 *)(gq + base + h * hs + (c - h * hd));
            continue;
        }
        const int kc = c - C;
        const float *g = kc < K * hd ? gk : gv;
        if (!g) continue;
        const int k2 = kc < K * hd ? kc : kc - K * hd;
        const int kvh = k2 / hd, d = k2 - kvh * hd;
        f4 s = {0.f, 0.f, 0.f, 0.f};
        for (int h = kvh * rep; h < (kvh + 1) * rep && h < H; ++h) s += *(const f4 *)(g + base + h * hs + d);
        row[f] = (beta ? row[f] : z) + s;
    }
}

extern "C" __global__ void __launch_bounds__(256)
heads_bwd_rows_k(const float *__restrict__ dy, float *__restrict__ dx, int T, int C, int H, int hd, int dir,
                 int beta) {
#pragma clang fp contract(off)
    int bt;
    int64_t base, hs;
    rows_bt(T, H, hd, bt, base, hs);
    for (int f = threadIdx.x; f < C / 4; f += 256) {
        const int c = 4 * f, h = c / hd;
        const int64_t o = base + h * hs + (c - h * hd);
        const f4 z = {0.f, 0.f, 0.f, 0.f};
        f4 *dst = (f4 *)(dx + (dir == 0 ? o : (int64_t)bt * C + c));
        const f4 src = *(const f4 *)(dy + (dir == 0 ? (int64_t)bt * C + c : o));
        *dst = (beta ? *dst : z) + src;
    }
}

// TOP_MERGE (train_tape.c:1329-1338): dctx[b,h,t,d] += dy[b,t,h*hd+d];
// TOP_HEADSPLIT (:1339-1350): dx[b,t,h*hd+d] += dy[b,h,t,d].  One thread
// per destination element.  dir 0: merge backward, 1: head-split backward.
extern "C" __global__ void __launch_bounds__(256)
heads_bwd_k(const float *__restrict__ dy, float *__restrict__ dx, int B, int T, int C, int H, int hd, int dir) {
#pragma clang fp contract(off)
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (dir == 0) {
        if (i >= (int64_t)B * H * T * hd) return;
        const int d = (int)(i % hd);
        const int t = (int)((i / hd) % T);
        const int64_t bh = i / ((int64_t)hd * T);
        const int h = (int)(bh % H), b = (int)(bh / H);
        if (h * hd + d < C) dx[i] += dy[((int64_t)b * T + t) * C + h * hd + d];
    } else {
        if (i >= (int64_t)B * T * C) return;
        const int c = (int)(i % C);
        const int64_t bt = i / C;
        const int t = (int)(bt % T), b = (int)(bt / T);
        const int h = c / hd, d = c - h * hd;
        if (h < H) dx[i] += dy[(((int64_t)b * H + h) * T + t) * hd + d];
    }
}

// TOP_SCALE backward (train_tape.c:1222-1231): dx += dy * s (float, two roundings)
extern "C" __global__ void __launch_bounds__(256)
axpy_k(float *__restrict__ dx, const float *__restrict__ dy, float s, int64_t n) {
#pragma clang fp contract(off)
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i < n) dx[i] = dx[i] + dy[i] * s;
}

// ---------------------------------------------------------------- recomputing (flash) backward
// The SDPA backward of the tape without stored probabilities: P is rebuilt
// tile by tile from q, k and each query row's softmax (max m, sum l) saved by
// the forward, P = exp(s scale + mask - m) / l, with the forward's own
// arithmetic.  D = rowsum(P o dP) is formed as rowsum(dO o O), its equal
// (sum_k P dP = sum_k P (dO . v_k) = dO . sum_k P v_k = dO . O).

// D[row] = sum_d dO[row][d] O[row][d] (fp64 sum), one wave per row, hd <= 64;
// row = (b H + h) T + t.  ldO > 0: O is stored with the heads merged, rows
// (b, t) of stride ldO and head h at column h hd.
extern "C" __global__ void __launch_bounds__(256)
sdpa_bwd_rowdot(const float *__restrict__ dO, const float *__restrict__ O, float *__restrict__ D, int64_t rows,
                int hd, int H, int T, int ldO) {
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= rows) return;
    int64_t oe = row * hd;
    if (ldO) {
        const int64_t bh = row / T, t = row - bh * T, b = bh / H, h = bh - b * H;
        oe = (b * T + t) * ldO + h * hd;
    }
    double s = lane < hd ? (double)dO[row * hd + lane] * (double)O[oe + lane] : 0.0;
    s = wave_sum_d(s);
    if (lane == 0) D[row] = (float)s;
}

// dq: 64 queries of one (b, h) per workgroup, wave w the queries q0 + 16w + li.
// Per key tile: S^T = K Q^T and dP^T = V dO^T in the layout (key 16c + 4g + r,
// query li), P and dS^T = P^T o (dP^T - D) in place, dq += dS K with dS^T as the
// A operand (as sdpa_bwd_dq_hd64's second sweep), one block of 16 keys at a
// time.  Causal: key tiles past the tile's last query are skipped (their P is
// exactly 0).  Under 128 registers (no prefetch of the next tile): four
// workgroups share a CU.
extern "C" __global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4, 4)))
sdpa_fbwd_dq_hd64(const float *__restrict__ q, const float *__restrict__ k, const float *__restrict__ v,
                  const float *__restrict__ mask, const float *__restrict__ stats, const float *__restrict__ D,
                  const float *__restrict__ dO, float *__restrict__ dq, int H, int Hkv, int Tq, int Tkv, float scale,
                  int causal, int beta, int ldo) {
    __shared__ __attribute__((aligned(16))) float sK[64 * SB_LD];
    __shared__ __attribute__((aligned(16))) float sV[64 * SB_LD];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int li = lane & 15, lg = lane >> 4;
    // grid (H, B, query tiles), the last query tile first: under a causal mask
    // it has the most key tiles, and dispatching the heaviest workgroups first
    // keeps the chip busy to the end (longest-first order)
    const int h = blockIdx.x, b = blockIdx.y;
    const int kvh = h / (H / Hkv);
    const int q0 = (gridDim.z - 1 - blockIdx.z) * 64, qw = q0 + wave * 16;
    const int my_q = qw + li;
    const int64_t rbase = ((int64_t)b * H + h) * Tq;
    const float *kb = k + ((int64_t)b * Hkv + kvh) * Tkv * 64;
    const float *vb = v + ((int64_t)b * Hkv + kvh) * Tkv * 64;
    const bool qok = my_q < Tq;

    f4 qf[4], gf[4];   // Q^T and dO^T fragments: query my_q, d = 16kc + 4g .. +3
#pragma unroll
    for (int kc = 0; kc < 4; ++kc) {
        qf[kc] = qok ? *(const f4 *)(q + (rbase + my_q) * 64 + kc * 16 + 4 * lg) : f4{0.f, 0.f, 0.f, 0.f};
        gf[kc] = qok ? *(const f4 *)(dO + (rbase + my_q) * 64 + kc * 16 + 4 * lg) : f4{0.f, 0.f, 0.f, 0.f};
    }
    const float mq = qok ? stats[(rbase + my_q) * 2] : 0.f;
    const float il = qok ? 1.0f / stats[(rbase + my_q) * 2 + 1] : 0.f;
    const float dq_d = qok ? D[rbase + my_q] : 0.f;
    f4 acc[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) acc[u] = f4{0.f, 0.f, 0.f, 0.f};

    const int coff = Tkv - Tq;
    int kend = Tkv;
    if (causal) kend = min(Tkv, q0 + 64 + coff);
    for (int k0 = 0; k0 < kend; k0 += 64) {
        __syncthreads();
        // all eight loads in flight at once (keys past Tkv read key Tkv - 1 and
        // are stored as zero), then the LDS stores (one LDS offset for the
        // thread's four rows, as in the dk / dv kernel)
        f4 vv[4], kk[4];
        const int r0 = tid >> 4, c0 = (tid & 15) * 4;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int64_t key = min(k0 + r0 + 16 * j, Tkv - 1);
            vv[j] = *(const f4 *)(vb + key * 64 + c0);
            kk[j] = *(const f4 *)(kb + key * 64 + c0);
        }
        const int so = r0 * SB_LD + LDS_SWZ(r0, c0);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const bool ok = k0 + r0 + 16 * j < Tkv;
            *(f4 *)(sV + so + 16 * j * SB_LD) = ok ? vv[j] : f4{0.f, 0.f, 0.f, 0.f};
            *(f4 *)(sK + so + 16 * j * SB_LD) = ok ? kk[j] : f4{0.f, 0.f, 0.f, 0.f};
        }
        __syncthreads();
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            f4 s = {0.f, 0.f, 0.f, 0.f}, dp = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int kc = 0; kc < 4; ++kc) {
                const f4 kf = *(const f4 *)(sK + (16 * c + li) * SB_LD + LDS_SWZ((16 * c + li), kc * 16 + 4 * lg));
                const f4 vf = *(const f4 *)(sV + (16 * c + li) * SB_LD + LDS_SWZ((16 * c + li), kc * 16 + 4 * lg));
#pragma unroll
                for (int st = 0; st < 4; ++st) {
                    s = mfma4(kf[st], qf[kc][st], s);
                    dp = mfma4(vf[st], gf[kc][st], dp);
                }
            }
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int key = k0 + 16 * c + 4 * lg + r;
                float x = s[r] * scale;
                if (mask && key < Tkv && qok) x += mask[(int64_t)my_q * Tkv + key];
                if (key >= Tkv || (causal && key > my_q + coff)) x = -INFINITY;
                const float p = qok ? __expf(x - mq) * il : 0.f;
                dp[r] = p * (dp[r] - dq_d);
            }
            // dq[query qw + 4g + r][d = 4li + u] += dS[query][key] K[key][d] over this block's keys
#pragma unroll
            for (int st = 0; st < 4; ++st) {
                const f4 kf = *(const f4 *)(sK + (16 * c + 4 * lg + st) * SB_LD + LDS_SWZ((16 * c + 4 * lg + st), 4 * li));
#pragma unroll
                for (int u = 0; u < 4; ++u) acc[u] = mfma4(dp[st], kf[u], acc[u]);
            }
        }
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int qi = qw + 4 * lg + r;
        if (qi < Tq) {
            // ldo > 0: rows (b, query) of stride ldo, head h at column 64 h
            f4 *o = (f4 *)(dq + (ldo ? ((int64_t)b * Tq + qi) * ldo + h * 64 : (rbase + qi) * 64) + 4 * li);
            f4 cur = beta ? *o : f4{0.f, 0.f, 0.f, 0.f};
            cur[0] += scale * acc[0][r];
            cur[1] += scale * acc[1][r];
            cur[2] += scale * acc[2][r];
            cur[3] += scale * acc[3][r];
            *o = cur;
        }
    }
}

// dk / dv: 64 keys of one (b, kv head) per workgroup, wave w the keys
// k0 + 16w + li.  For every query head of the group and query tile, per block
// of 16 queries c: S = Q K^T and dP = dO V^T in the layout (query 16c + 4g +
// r, key li), P and dS in registers (no transposed copy of P), then at once
// dV += P^T dO and dK += dS^T Q for that block, so only one block's P and dS
// are live.  Causal: query tiles before the first query that sees this key
// tile are skipped.  No register prefetch of the next tile: the registers
// stay under 128, so four workgroups share a CU and hide each other's loads.
extern "C" __global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4, 4)))
sdpa_fbwd_dkdv_hd64(const float *__restrict__ q, const float *__restrict__ k, const float *__restrict__ v,
                    const float *__restrict__ mask, const float *__restrict__ stats, const float *__restrict__ D,
                    const float *__restrict__ dO, float *__restrict__ dk, float *__restrict__ dv, int H, int Hkv,
                    int Tq, int Tkv, float scale, int causal, int beta, int ldo) {
    __shared__ __attribute__((aligned(16))) float sG[64 * SB_LD];   // dO tile [query][d]
    __shared__ __attribute__((aligned(16))) float sQ[64 * SB_LD];   // Q tile  [query][d]
    __shared__ __attribute__((aligned(16))) float sM[64];
    __shared__ __attribute__((aligned(16))) float sL[64];
    __shared__ __attribute__((aligned(16))) float sD[64];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int li = lane & 15, lg = lane >> 4;
    // grid (Hkv, B, key tiles), the first key tile first: under a causal mask
    // it meets the most query tiles, and dispatching the heaviest workgroups
    // first keeps the chip busy to the end (longest-first order)
    const int kvh = blockIdx.x, b = blockIdx.y;
    const int rep = H / Hkv;
    const int k0 = blockIdx.z * 64;
    const int kl = wave * 16 + li;
    const int my_k = k0 + kl;
    const bool kok = my_k < Tkv;
    const int64_t kbase = ((int64_t)b * Hkv + kvh) * Tkv;

    f4 vf[4], kf[4];   // V and K fragments: key my_k, d = 16kc + 4g .. +3
#pragma unroll
    for (int kc = 0; kc < 4; ++kc) {
        vf[kc] = kok ? *(const f4 *)(v + (kbase + my_k) * 64 + kc * 16 + 4 * lg) : f4{0.f, 0.f, 0.f, 0.f};
        kf[kc] = kok ? *(const f4 *)(k + (kbase + my_k) * 64 + kc * 16 + 4 * lg) : f4{0.f, 0.f, 0.f, 0.f};
    }
    f4 ak[4], av[4];   // [u][r]: key k0 + 16w + 4g + r, d = 4li + u
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        ak[u] = f4{0.f, 0.f, 0.f, 0.f};
        av[u] = f4{0.f, 0.f, 0.f, 0.f};
    }
    const int coff = Tkv - Tq;
    int qstart = 0;
    if (causal) {   // the first query that sees key k0 is k0 - coff
        const int first = k0 - coff;
        qstart = first > 0 ? (first / 64) * 64 : 0;
    }
    // the (query head, query tile) pairs in order
    const int nq = qstart < Tq ? (Tq - qstart + 63) / 64 : 0, niter = rep * nq;
    for (int it = 0; it < niter; ++it) {
        const int h = kvh * rep + it / nq, q0 = qstart + (it % nq) * 64;
        const int64_t rbase = ((int64_t)b * H + h) * Tq;
        __syncthreads();
        // all eight loads in flight at once (rows past Tq read row Tq - 1 and
        // are stored as zero), then the LDS stores.  Thread tid stages rows
        // tid / 16 + 16 j, columns 4 (tid % 16): the swizzle depends on bits 2
        // and 3 of the row only, so one LDS offset serves all four rows.
        f4 g[4], qq[4];
        const int r0 = tid >> 4, c0 = (tid & 15) * 4;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int64_t qr = rbase + min(q0 + r0 + 16 * j, Tq - 1);
            g[j] = *(const f4 *)(dO + qr * 64 + c0);
            qq[j] = *(const f4 *)(q + qr * 64 + c0);
        }
        const int so = r0 * SB_LD + LDS_SWZ(r0, c0);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const bool ok = q0 + r0 + 16 * j < Tq;
            *(f4 *)(sG + so + 16 * j * SB_LD) = ok ? g[j] : f4{0.f, 0.f, 0.f, 0.f};
            *(f4 *)(sQ + so + 16 * j * SB_LD) = ok ? qq[j] : f4{0.f, 0.f, 0.f, 0.f};
        }
        if (tid < 64) {
            const int qi = q0 + tid;
            const bool ok = qi < Tq;
            sM[tid] = ok ? stats[(rbase + qi) * 2] : 0.f;
            sL[tid] = ok ? 1.0f / stats[(rbase + qi) * 2 + 1] : 0.f;
            sD[tid] = ok ? D[rbase + qi] : 0.f;
        }
        __syncthreads();
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            f4 dp = {0.f, 0.f, 0.f, 0.f}, s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int kc = 0; kc < 4; ++kc) {
                const f4 gfr = *(const f4 *)(sG + (16 * c + li) * SB_LD + LDS_SWZ((16 * c + li), kc * 16 + 4 * lg));
                const f4 qfr = *(const f4 *)(sQ + (16 * c + li) * SB_LD + LDS_SWZ((16 * c + li), kc * 16 + 4 * lg));
#pragma unroll
                for (int st = 0; st < 4; ++st) {
                    dp = mfma4(gfr[st], vf[kc][st], dp);
                    s = mfma4(qfr[st], kf[kc][st], s);
                }
            }
            const f4 mm = *(const f4 *)(sM + 16 * c + 4 * lg);
            const f4 ll = *(const f4 *)(sL + 16 * c + 4 * lg);
            const f4 dd = *(const f4 *)(sD + 16 * c + 4 * lg);
            f4 pf;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int qi = q0 + 16 * c + 4 * lg + r;
                float x = s[r] * scale;
                if (mask && qi < Tq && kok) x += mask[(int64_t)qi * Tkv + my_k];
                if (!kok || (causal && my_k > qi + coff)) x = -INFINITY;
                const float p = qi < Tq ? __expf(x - mm[r]) * ll[r] : 0.f;
                pf[r] = p;
                dp[r] = p * (dp[r] - dd[r]);
            }
            // dV += P^T dO, dK += dS^T Q over this block's 16 queries
#pragma unroll
            for (int st = 0; st < 4; ++st) {
                const f4 gfr = *(const f4 *)(sG + (16 * c + 4 * lg + st) * SB_LD + LDS_SWZ((16 * c + 4 * lg + st), 4 * li));
                const f4 qfr = *(const f4 *)(sQ + (16 * c + 4 * lg + st) * SB_LD + LDS_SWZ((16 * c + 4 * lg + st), 4 * li));
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    av[u] = mfma4(pf[st], gfr[u], av[u]);
                    ak[u] = mfma4(dp[st], qfr[u], ak[u]);
                }
            }
        }
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int key = k0 + wave * 16 + 4 * lg + r;
        if (key < Tkv) {
            // ldo > 0: rows (b, key) of stride ldo, kv head kvh at column 64 kvh
            const int64_t oe = (ldo ? ((int64_t)b * Tkv + key) * ldo + kvh * 64 : (kbase + key) * 64) + 4 * li;
            if (dk) {
                f4 *o = (f4 *)(dk + oe);
                f4 cur = beta ? *o : f4{0.f, 0.f, 0.f, 0.f};
                cur[0] += scale * ak[0][r];
                cur[1] += scale * ak[1][r];
                cur[2] += scale * ak[2][r];
                cur[3] += scale * ak[3][r];
                *o = cur;
            }
            if (dv) {
                f4 *o = (f4 *)(dv + oe);
                f4 cur = beta ? *o : f4{0.f, 0.f, 0.f, 0.f};
                cur[0] += av[0][r];
                cur[1] += av[1][r];
                cur[2] += av[2][r];
                cur[3] += av[3][r];
                *o = cur;
            }
        }
    }
}
