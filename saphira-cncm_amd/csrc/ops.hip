// ops.hip -- row-wise and elementwise kernels around the GEMMs.
#include "mfma_slab.h"

// Greedy id: per row the reference's strict '>' scan from index 0
// (kernels.c:731-735): index 0 when x[0] is NaN, otherwise the lowest index
// of the maximal non-NaN value (0 when no value exceeds x[0] = -inf).
extern "C" __global__ void __launch_bounds__(256)
argmax_rows_k(const float *__restrict__ x, int n, int *__restrict__ idx) {
    __shared__ float bv[4];
    __shared__ int bi[4];
    const int tid = threadIdx.x;
    const float *xr = x + (int64_t)blockIdx.x * n;
    float best = -INFINITY;
    int bidx = 0x7fffffff;
    for (int j = tid; j < n; j += 256) {
        float v = xr[j];
        if (v > best) { best = v; bidx = j; }
    }
    for (int o = 32; o > 0; o >>= 1) {
        float ov = __shfl_xor(best, o, 64);
        int oi = __shfl_xor(bidx, o, 64);
        if (ov > best || (ov == best && oi < bidx)) { best = ov; bidx = oi; }
    }
    if ((tid & 63) == 0) { bv[tid >> 6] = best; bi[tid >> 6] = bidx; }
    __syncthreads();
    if (tid == 0) {
        float b = bv[0];
        int i = bi[0];
        for (int w = 1; w < 4; ++w)
            if (bv[w] > b || (bv[w] == b && bi[w] < i)) { b = bv[w]; i = bi[w]; }
        float x0 = xr[0];
        if (x0 != x0 || i == 0x7fffffff) i = 0;
        idx[blockIdx.x] = i;
    }
}

// ---------------------------------------------------------------- norms
// RMSNorm (kernels.c:150-162): ms = sum x^2 in fp64 / C, s = (float)(1/sqrt(ms
// + 1e-6)), y = (x*s)*w in float.  LayerNorm (kernels.c:101-148): mean and
// var in fp64, y = (float)((x-mean)*inv)*w + b in float.  One wave per row;
// the fp64 sums are tree-ordered (the reference sums serially), the float
// arithmetic after the statistics follows the reference's roundings.
extern "C" __global__ void __launch_bounds__(256)
rmsnorm_k(const float *__restrict__ x, const float *__restrict__ w, float *__restrict__ y, int64_t rows, int C) {
#pragma clang fp contract(off)
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= rows) return;
    const float *xr = x + row * C;
    double ms = 0.0;
    for (int c = lane; c < C; c += 64) ms += (double)xr[c] * (double)xr[c];
    ms = wave_sum_d(ms) / C;
    const float s = (float)(1.0 / sqrt(ms + 1e-6));
    float *yr = y + row * C;
    for (int c = lane; c < C; c += 64) yr[c] = xr[c] * s * (w ? w[c] : 1.0f);
}

extern "C" __global__ void __launch_bounds__(256)
layernorm_k(const float *__restrict__ x, const float *__restrict__ w, const float *__restrict__ b,
            float *__restrict__ y, int64_t rows, int C, double eps) {
#pragma clang fp contract(off)
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= rows) return;
    const float *xr = x + row * C;
    double mean = 0.0;
    for (int c = lane; c < C; c += 64) mean += (double)xr[c];
    mean = wave_sum_d(mean) / C;
    double var = 0.0;
    for (int c = lane; c < C; c += 64) {
        double d = (double)xr[c] - mean;
        var += d * d;
    }
    var = wave_sum_d(var) / C;
    const double inv = 1.0 / sqrt(var + eps);
    float *yr = y + row * C;
    for (int c = lane; c < C; c += 64)
        yr[c] = (float)(((double)xr[c] - mean) * inv) * (w ? w[c] : 1.0f) + (b ? b[c] : 0.0f);
}

// Register-resident forms of rmsnorm_k (KIND 1) and layernorm_k (KIND 0) for
// C <= 256 * NPL, C % 4 == 0 and 16-byte aligned rows: the wave reads its row
// once as float4 groups (group q = lane + 64 j) with every load in flight,
// and the statistics and the output come from those registers, with the
// kernels' arithmetic per element.  In place (y == x) is allowed: a row is
// read whole before it is written.
template <int KIND, int NPL>
__device__ __forceinline__ void norm_rows4(const float *x, const float *__restrict__ w, const float *__restrict__ b,
                                           float *y, int64_t rows, int C, double eps) {
#pragma clang fp contract(off)
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= rows) return;
    f4 v[NPL];
#pragma unroll
    for (int j = 0; j < NPL; ++j) {
        const int c = 4 * (lane + 64 * j);
        v[j] = c < C ? *(const f4 *)(x + row * C + c) : f4{0.f, 0.f, 0.f, 0.f};
    }
    if (KIND == 0) {
        double mean = 0.0;
#pragma unroll
        for (int j = 0; j < NPL; ++j)
#pragma unroll
            for (int e = 0; e < 4; ++e) mean += (double)v[j][e];
        mean = wave_sum_d(mean) / C;
        double var = 0.0;
#pragma unroll
        for (int j = 0; j < NPL; ++j)
            if (4 * (lane + 64 * j) < C)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const double d = (double)v[j][e] - mean;
                    var += d * d;
                }
        var = wave_sum_d(var) / C;
        const double inv = 1.0 / sqrt(var + eps);
#pragma unroll
        for (int j = 0; j < NPL; ++j) {
            const int c = 4 * (lane + 64 * j);
            if (c >= C) continue;
            const f4 wv = w ? *(const f4 *)(w + c) : f4{1.f, 1.f, 1.f, 1.f};
            const f4 bv = b ? *(const f4 *)(b + c) : f4{0.f, 0.f, 0.f, 0.f};
            f4 o;
#pragma unroll
            for (int e = 0; e < 4; ++e) o[e] = (float)(((double)v[j][e] - mean) * inv) * wv[e] + bv[e];
            *(f4 *)(y + row * C + c) = o;
        }
    } else {
        double ms = 0.0;
#pragma unroll
        for (int j = 0; j < NPL; ++j)
#pragma unroll
            for (int e = 0; e < 4; ++e) ms += (double)v[j][e] * (double)v[j][e];
        ms = wave_sum_d(ms) / C;
        const float s = (float)(1.0 / sqrt(ms + 1e-6));
#pragma unroll
        for (int j = 0; j < NPL; ++j) {
            const int c = 4 * (lane + 64 * j);
            if (c >= C) continue;
            const f4 wv = w ? *(const f4 *)(w + c) : f4{1.f, 1.f, 1.f, 1.f};
            f4 o;
#pragma unroll
            for (int e = 0; e < 4; ++e) o[e] = v[j][e] * s * wv[e];
            *(f4 *)(y + row * C + c) = o;
        }
    }
}

#define NORM_ROWS4(name, KIND, NPL)                                                                            \
    extern "C" __global__ void __launch_bounds__(256)                                                         \
        name(const float *x, const float *__restrict__ w, const float *__restrict__ b, float *y, int64_t rows, \
             int C, double eps) {                                                                             \
        norm_rows4<KIND, NPL>(x, w, b, y, rows, C, eps);                                                      \
    }
NORM_ROWS4(layernorm4_1, 0, 1)
NORM_ROWS4(layernorm4_2, 0, 2)
NORM_ROWS4(layernorm4_3, 0, 3)
NORM_ROWS4(layernorm4_4, 0, 4)
NORM_ROWS4(rmsnorm4_1, 1, 1)
NORM_ROWS4(rmsnorm4_2, 1, 2)
NORM_ROWS4(rmsnorm4_3, 1, 3)
NORM_ROWS4(rmsnorm4_4, 1, 4)

// ---------------------------------------------------------------- RoPE
// Rotate-half RoPE in place (kernels.c:249-264): rows of hd, position
// row % T, y[d] = a*c[d] + (-b)*s[d], y[d+h] = b*c[d+h] + a*s[d+h] with the
// reference's separate roundings.  One thread per (row, d < hd/2).
extern "C" __global__ void __launch_bounds__(256)
rope_k(float *x, const float *__restrict__ cos_t, const float *__restrict__ sin_t, int64_t rows, int T, int hd) {
#pragma clang fp contract(off)
    const int h = hd >> 1;
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= rows * h) return;
    const int64_t row = i / h;
    const int d = (int)(i % h);
    const int t = (int)(row % T);
    float *xr = x + row * hd;
    const float *co = cos_t + (int64_t)t * hd, *si = sin_t + (int64_t)t * hd;
    const float a = xr[d], bb = xr[d + h];
    xr[d] = a * co[d] + (-bb) * si[d];
    xr[d + h] = bb * co[d + h] + a * si[d + h];
}

// ---------------------------------------------------------------- layout
// heads_transpose_fwd_b (kernels.c:345-357): [B][T][H*hd] -> [B][H][T][hd]
extern "C" __global__ void __launch_bounds__(256)
heads_transpose_k(const float *__restrict__ in, float *__restrict__ out, int B, int64_t T, int H, int hd) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t n = (int64_t)B * T * H * hd;
    if (i >= n) return;
    const int d = (int)(i % hd);
    const int64_t t = (i / hd) % T;
    const int64_t bh = i / ((int64_t)hd * T);
    const int h = (int)(bh % H), b = (int)(bh / H);
    out[i] = in[(((int64_t)b * T + t) * H + h) * hd + d];
}

// qkv_split_fwd (kernels.c:891-926): fused qkv rows -> q, k, v heads (GQA
// replication kv head = h / rep)
extern "C" __global__ void __launch_bounds__(256)
qkv_split_k(const float *__restrict__ in, float *__restrict__ qq, float *__restrict__ kk, float *__restrict__ vv,
            int B, int T, int C, int H, int hd, int K, int rep) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (int64_t)B * H * T * hd) return;
    const int d = (int)(i % hd);
    const int t = (int)((i / hd) % T);
    const int h = (int)((i / ((int64_t)hd * T)) % H);
    const int b = (int)(i / ((int64_t)H * T * hd));
    const int kvh = h / rep;
    const float *row = in + ((int64_t)b * T + t) * ((int64_t)C + 2 * K * hd);
    qq[i] = row[h * hd + d];
    kk[i] = row[C + kvh * hd + d];
    vv[i] = row[C + K * hd + kvh * hd + d];
}

// qkv_split_fwd followed by rope_apply on q and k (kernels.c:913-926,
// 285-296), one thread per rotation pair (d, d + hd/2) of one (b, h, t): the
// rotation repeats rope_k's float operations on the values qkv_split_k would
// have written.
extern "C" __global__ void __launch_bounds__(256)
qkv_split_rope_k(const float *__restrict__ in, float *__restrict__ qq, float *__restrict__ kk,
                 float *__restrict__ vv, const float *__restrict__ cos_t, const float *__restrict__ sin_t, int B,
                 int T, int C, int H, int hd, int K, int rep) {
#pragma clang fp contract(off)
    const int h2 = hd >> 1;
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (int64_t)B * H * T * h2) return;
    const int d = (int)(i % h2);
    const int64_t row = i / h2;   // [B][H][T] row
    const int t = (int)(row % T);
    const int h = (int)((row / T) % H);
    const int b = (int)(row / ((int64_t)T * H));
    const int kvh = h / rep;
    const float *src = in + ((int64_t)b * T + t) * ((int64_t)C + 2 * K * hd);
    const float *co = cos_t + (int64_t)t * hd, *si = sin_t + (int64_t)t * hd;
    float *qr = qq + row * hd, *kr = kk + row * hd, *vr = vv + row * hd;
    const float qa = src[h * hd + d], qb = src[h * hd + d + h2];
    qr[d] = qa * co[d] + (-qb) * si[d];
    qr[d + h2] = qb * co[d + h2] + qa * si[d + h2];
    const float ka = src[C + kvh * hd + d], kb = src[C + kvh * hd + d + h2];
    kr[d] = ka * co[d] + (-kb) * si[d];
    kr[d + h2] = kb * co[d + h2] + ka * si[d + h2];
    vr[d] = src[C + K * hd + kvh * hd + d];
    vr[d + h2] = src[C + K * hd + kvh * hd + d + h2];
}

// head_merge_fwd (kernels.c:903-936): [B][H][T][hd] -> [B][T][C]
extern "C" __global__ void __launch_bounds__(256)
head_merge_k(const float *__restrict__ ctx, float *__restrict__ out, int B, int T, int C, int H, int hd) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (int64_t)B * T * C) return;
    const int c = (int)(i % C);
    const int hh = c / hd, dd = c % hd;
    const int t = (int)((i / C) % T);
    const int b = (int)(i / ((int64_t)T * C));
    out[i] = ctx[(((int64_t)b * H + hh) * T + t) * hd + dd];
}

// Row-blocked forms of the three layout kernels above, for hd and C multiples
// of 4 and 16-byte aligned operands: one workgroup per (b, t) row and one
// float4 per thread and pass, so the row's index arithmetic is done once per
// workgroup in 32-bit (the per-element forms spend most of their time in
// 64-bit division) and every access is 16 bytes inside a run of hd floats.
// Head h of row (b, t) in a [B][H][T][hd] tensor starts at base + h * hs.
__device__ __forceinline__ void row_bt(int T, int H, int hd, int &bt, int64_t &base, int64_t &hs) {
    bt = blockIdx.x;
    const int b = bt / T, t = bt - b * T;
    hs = (int64_t)T * hd;
    base = ((int64_t)b * H * T + t) * hd;
}

extern "C" __global__ void __launch_bounds__(256)
qkv_split_rows_k(const float *__restrict__ in, float *__restrict__ qq, float *__restrict__ kk,
                 float *__restrict__ vv, int T, int C, int H, int hd, int K, int rep) {
    int bt;
    int64_t base, hs;
    row_bt(T, H, hd, bt, base, hs);
    const int rl = C + 2 * K * hd;
    const f4 *row = (const f4 *)(in + (int64_t)bt * rl);
    for (int f = threadIdx.x; f < rl / 4; f += 256) {
        const int c = 4 * f;
        const f4 v = row[f];
        if (c < C) {
            const int h = c / hd;
            if (h < H) *(f4 *)(qq + base + h * hs + (c - h * hd)) = v;
        } else {
            // kv head kvh feeds query heads kvh * rep .. kvh * rep + rep - 1
            const int kc = c - C;
            float *dst = kc < K * hd ? kk : vv;
            const int k2 = kc < K * hd ? kc : kc - K * hd;
            const int kvh = k2 / hd, d = k2 - kvh * hd;
            for (int h = kvh * rep; h < (kvh + 1) * rep && h < H; ++h) *(f4 *)(dst + base + h * hs + d) = v;
        }
    }
}

extern "C" __global__ void __launch_bounds__(256)
head_merge_rows_k(const float *__restrict__ ctx, float *__restrict__ out, int T, int C, int H, int hd) {
    int bt;
    int64_t base, hs;
    row_bt(T, H, hd, bt, base, hs);
    f4 *orow = (f4 *)(out + (int64_t)bt * C);
    for (int f = threadIdx.x; f < C / 4; f += 256) {
        const int c = 4 * f, h = c / hd;
        orow[f] = *(const f4 *)(ctx + base + h * hs + (c - h * hd));
    }
}

extern "C" __global__ void __launch_bounds__(256)
heads_transpose_rows_k(const float *__restrict__ in, float *__restrict__ out, int T, int H, int hd) {
    int bt;
    int64_t base, hs;
    row_bt(T, H, hd, bt, base, hs);
    const f4 *irow = (const f4 *)(in + (int64_t)bt * H * hd);
    for (int f = threadIdx.x; f < H * hd / 4; f += 256) {
        const int c = 4 * f, h = c / hd;
        *(f4 *)(out + base + h * hs + (c - h * hd)) = irow[f];
    }
}

// A prefill's q, k, v rows (from their GEMMs, [T][H hd] and [T][K hd]) to
// attention layout with RoPE, and k, v into the KV cache: one workgroup per
// position t, one rotation pair (d, d + hd/2) per thread and pass.  The
// operations are heads_transpose_fwd's copies and rope_k's float operations
// (y[d] = a c[d] + (-b) s[d], y[d + h] = b c[d + h] + a s[d + h]); qq
// [H][T][hd], kk / vv [K][T][hd], kc / vc [K][ld][hd] at row t.
extern "C" __global__ void __launch_bounds__(256)
qkv_rope_cache_k(const float *__restrict__ ql, const float *__restrict__ kl, const float *__restrict__ vl,
                 float *__restrict__ qq, float *__restrict__ kk, float *__restrict__ vv, float *__restrict__ kc,
                 float *__restrict__ vc, const float *__restrict__ cos_t, const float *__restrict__ sin_t, int T,
                 int H, int K, int hd, int ld) {
#pragma clang fp contract(off)
    const int t = blockIdx.x, h2 = hd >> 1;
    const float *co = cos_t + (int64_t)t * hd, *si = sin_t + (int64_t)t * hd;
    // q and k rotation pairs: H + K heads of h2 pairs; then v: K heads of hd
    for (int i = threadIdx.x; i < (H + K) * h2; i += 256) {
        const int hh = i / h2, d = i - hh * h2;
        const bool isq = hh < H;
        const int head = isq ? hh : hh - H;
        const float *src = isq ? ql + ((int64_t)t * H + head) * hd : kl + ((int64_t)t * K + head) * hd;
        const float a = src[d], b = src[d + h2];
        const float y0 = a * co[d] + (-b) * si[d];
        const float y1 = b * co[d + h2] + a * si[d + h2];
        float *dst = isq ? qq + ((int64_t)head * T + t) * hd : kk + ((int64_t)head * T + t) * hd;
        dst[d] = y0;
        dst[d + h2] = y1;
        if (!isq) {
            float *c = kc + ((int64_t)head * ld + t) * hd;
            c[d] = y0;
            c[d + h2] = y1;
        }
    }
    for (int i = threadIdx.x; i < K * hd; i += 256) {
        const int head = i / hd, d = i - head * hd;
        const float x = vl[((int64_t)t * K + head) * hd + d];
        vv[((int64_t)head * T + t) * hd + d] = x;
        vc[((int64_t)head * ld + t) * hd + d] = x;
    }
}

// embedding_fwd (kernels.c:59-74): y[i,:] = W[idx[i],:]; ids outside [0, V)
// read row 0 (the reference would read out of bounds).
extern "C" __global__ void __launch_bounds__(256)
embedding_k(const float *__restrict__ W, const int *__restrict__ idx, float *__restrict__ y, int64_t n, int D, int V) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n * D) return;
    int id = idx[i / D];
    if ((unsigned)id >= (unsigned)V) id = 0;
    y[i] = W[(int64_t)id * D + (i % D)];
}

// ---------------------------------------------------------------- elementwise
// op: 0 add (a+b), 1 mul (a*b), 2 scale (a*s), 3 add_inplace (y += a),
//     4 silu, 5 gelu, 6 gelu_tanh   (kernels.c:167-226, 829-874),
//     7 y = 0.0f + a (add_inplace into a fresh gradient: the bits of
//       accumulating into zeros, without reading or clearing y)
__device__ __forceinline__ float elt_op(float v, float w, float yv, float s, int op) {
#pragma clang fp contract(off)
    switch (op) {
    case 0: return v + w;
    case 1: return v * w;
    case 2: return v * s;
    case 3: return yv + v;
    case 7: return 0.0f + v;
    case 4: return ncm_act(v, ACT_SILU);
    case 5: return ncm_act(v, ACT_GELU);
    default: return ncm_act(v, ACT_GELU_TANH);
    }
}

extern "C" __global__ void __launch_bounds__(256)
eltwise_k(const float *a, const float *b, float *y, float s, int64_t n, int op) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    y[i] = elt_op(a[i], (op == 0 || op == 1) ? b[i] : 0.f, op == 3 ? y[i] : 0.f, s, op);
}

// The same on float4 groups (n4 = n / 4, 16-byte aligned operands): each
// element gets the scalar kernel's float operations; a, b and y may alias
// (each element is read before it is written, by the same thread).
extern "C" __global__ void __launch_bounds__(256)
eltwise4_k(const float *a, const float *b, float *y, float s, int64_t n4, int op) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n4) return;
    const f4 v = ((const f4 *)a)[i];
    const f4 w = (op == 0 || op == 1) ? ((const f4 *)b)[i] : f4{0.f, 0.f, 0.f, 0.f};
    const f4 yv = op == 3 ? ((const f4 *)y)[i] : f4{0.f, 0.f, 0.f, 0.f};
    f4 r;
#pragma unroll
    for (int e = 0; e < 4; ++e) r[e] = elt_op(v[e], w[e], yv[e], s, op);
    ((f4 *)y)[i] = r;
}

// ---------------------------------------------------------------- SDPA
// softmax(Q K^T * scale + mask) V with GQA (kernels.c:364-507), q [B][Hq][Tq][hd],
// k/v [B][Hkv][Tkv][hd], out like q, kv head = h / (Hq/Hkv), mask [Tq][Tkv]
// additive (or null).  causal: query tq sees keys <= tq + (Tkv - Tq) (the
// bottom-right alignment a KV cache needs; the usual mask when Tq == Tkv).
//
// sdpa_hd64: flash-style, FP32 MFMA.  A workgroup owns 64 queries of one
// (b, h); each wave 16.  Per 64-key tile staged in LDS:
//   S^T = K Q^T   (so the accumulator of lane (li, g) holds the scores of
//                  query li for keys 16c + 4g + r -- exactly the A operand
//                  of the next product under the k-permutation below);
//   online softmax per query (running max m, sum l, rescale of O);
//   O += P V.
// k-permutation as in the GEMM: MFMA step s gives lane group g the reduction
// index 4g + s (d for S^T, key for P V).  Q stays in registers.
#define SD_T 64
// LDS slot of float4 group g (0..15) of row r in the 64-float rows of the
// flash kernels' K / V tiles (an involution in g for each r)
__device__ __forceinline__ int sd_slot(int r, int g) { return g ^ (r & 15) ^ (((r >> 2) & 1) << 3); }

// The loop of one workgroup: queries q0 .. q0 + 63 of (b, h) over the key
// blocks [kb_lo, kb_hi) (64 keys each) of the range the query tile sees.
// part_o == nullptr: the whole range -- the output is normalised and stored
// (and the row statistics when asked for); otherwise a part of a split range:
// the unnormalised O rows and each query's (max, sum) go to the part's slot
// for sdpa_hd64_combine.
__device__ __forceinline__ void sdpa_hd64_body(const float *__restrict__ q, const float *__restrict__ k,
                                               const float *__restrict__ v, const float *__restrict__ mask,
                                               float *__restrict__ out, int Hq, int Hkv, int Tq, int Tkv,
                                               float scale, int causal, int merged, float *__restrict__ stats,
                                               int h, int b, int q0, int kb_lo, int kb_hi,
                                               float *__restrict__ part_o, float *__restrict__ part_ml,
                                               int64_t mask_bs) {
    // K and V tiles of 64 keys x 64 d, unpadded, float4 group g of key row r
    // in slot sd_slot(r, g).  A gfx950 ds_read_b128 serves lanes {0-3, 12-15,
    // 20-23, 24-27} (or {4-7, 8-11, 16-19, 28-31}) together: S^T's reads
    // (lane li: row 16c + li, group 4kc + lg) and P V's (lane li: row
    // 16c + 4lg + st, group li) then meet 16 different slots; with the plain
    // g ^ (r & 15) the P V rows r and r + 4 collided.
    __shared__ __attribute__((aligned(16))) float sK[SD_T * 64];
    if (mask) mask += (int64_t)b * mask_bs;   // a board's own mask (mask_bs 0: one mask for all)
    __shared__ __attribute__((aligned(16))) float sV[SD_T * 64];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int li = lane & 15, lg = lane >> 4;
    const int kvh = h / (Hq / Hkv);
    const int qw = q0 + wave * 16;
    const float *qb = q + ((int64_t)b * Hq + h) * Tq * 64;
    const float *kb = k + ((int64_t)b * Hkv + kvh) * Tkv * 64;
    const float *vb = v + ((int64_t)b * Hkv + kvh) * Tkv * 64;
    // Tiles go from L2 straight into LDS (buffer_load_dwordx4 ... lds):
    // load e of wave w fills key rows 4 (4w + e) .. +3, lane l row
    // 4 (4w + e) + l / 16, slot l % 16; rows past Tkv lie beyond the buffer
    // and read zero.
    const __amdgpu_buffer_rsrc_t rk = make_rsrc(kb, (unsigned)Tkv * 256u), rv = make_rsrc(vb, (unsigned)Tkv * 256u);
    const int lrow = lane >> 4, lslot = lane & 15;
    auto issue = [&](__amdgpu_buffer_rsrc_t rs, float *dst, int k0) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int r = 4 * (4 * wave + e) + lrow;
            const unsigned off = (unsigned)(k0 + r) * 256u + 16u * (unsigned)sd_slot(r, lslot);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                rs, (__attribute__((address_space(3))) void *)(dst + (4 * wave + e) * 256), 16, off, 0, 0, 0);
        }
    };

    // Q^T fragments: query qw + li, d = 16kc + 4g .. +3
    f4 qf[4];
#pragma unroll
    for (int kc = 0; kc < 4; ++kc) {
        const int qi = qw + li;
        qf[kc] = qi < Tq ? *(const f4 *)(qb + (int64_t)qi * 64 + kc * 16 + 4 * lg) : f4{0.f, 0.f, 0.f, 0.f};
    }
    const int my_q = qw + li;                 // query of this lane in the S^T layout
    float m_run = -INFINITY, l_run = 0.f;     // per query my_q (replicated over lg)
    f4 o[4];                                  // o[u][r]: query qw + 4lg + r, d = 4li + u
#pragma unroll
    for (int u = 0; u < 4; ++u) o[u] = f4{0.f, 0.f, 0.f, 0.f};

    const int coff = Tkv - Tq;   // causal offset of the query positions
    int kend = Tkv;
    if (causal) kend = min(Tkv, q0 + 64 + coff);
    // Per key tile, two barriers: (1) after S^T and the softmax, once this
    // wave's V loads have landed: every wave is done reading K and every V
    // row is in LDS, so the next tile's K loads go out (overlapping P V);
    // (2) after P V, once the next K has landed: V is free and the next K
    // is in LDS, so the next V loads go out (overlapping the next S^T and
    // softmax).
    kend = min(kend, kb_hi * SD_T);
    const int kfirst = kb_lo * SD_T;
    if (kfirst < kend) {
        issue(rk, sK, kfirst);
        issue(rv, sV, kfirst);
    }
    __builtin_amdgcn_s_waitcnt(0x0f70);   // vmcnt(0)
    __syncthreads();
    for (int k0 = kfirst; k0 < kend; k0 += SD_T) {
        const bool more = k0 + SD_T < kend;
        // S^T[c]: keys k0 + 16c + 4lg + r, query my_q
        f4 s[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            s[c] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int kc = 0; kc < 4; ++kc) {
                const f4 kf = *(const f4 *)(sK + (16 * c + li) * 64 + 4 * sd_slot(16 * c + li, 4 * kc + lg));
#pragma unroll
                for (int st = 0; st < 4; ++st) s[c] = mfma4(kf[st], qf[kc][st], s[c]);
            }
        }
        // scale, mask, tile max
        float mt = -INFINITY;
#pragma unroll
        for (int c = 0; c < 4; ++c)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int key = k0 + 16 * c + 4 * lg + r;
                float x = s[c][r] * scale;
                if (mask && key < Tkv && my_q < Tq) x += mask[(int64_t)my_q * Tkv + key];
                if (key >= Tkv || (causal && key > my_q + coff)) x = -INFINITY;
                s[c][r] = x;
                mt = fmaxf(mt, x);
            }
        mt = fmaxf(mt, __shfl_xor(mt, 16, 64));
        mt = fmaxf(mt, __shfl_xor(mt, 32, 64));
        const float m_new = fmaxf(m_run, mt);
        const bool none = m_new == -INFINITY;     // every key so far masked
        const float alpha = none ? 1.f : __expf(m_run - m_new);
        float ps = 0.f;
#pragma unroll
        for (int c = 0; c < 4; ++c)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float p = none ? 0.f : __expf(s[c][r] - m_new);
                s[c][r] = p;
                ps += p;
            }
        ps += __shfl_xor(ps, 16, 64);
        ps += __shfl_xor(ps, 32, 64);
        l_run = l_run * alpha + ps;
        m_run = m_new;
        // every wave is done reading K and this tile's V is in LDS: the next
        // K loads go out, overlapping P V (issued after the mask's loads,
        // which the softmax has waited for)
        __builtin_amdgcn_s_waitcnt(0x0f70);   // vmcnt(0): this wave's V loads
        __syncthreads();
        __builtin_amdgcn_sched_barrier(0);
        if (more) issue(rk, sK, k0 + SD_T);
        __builtin_amdgcn_sched_barrier(0);
        // rescale O rows (query qw + 4lg + r) by the alpha held in lane li = 4lg + r
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const float ar = __shfl(alpha, 4 * lg + r, 64);
#pragma unroll
            for (int u = 0; u < 4; ++u) o[u][r] *= ar;
        }
        // O += P V: chunk c, step st -> key 16c + 4lg + st; V float4 along d = 4li..
#pragma unroll
        for (int c = 0; c < 4; ++c)
#pragma unroll
            for (int st = 0; st < 4; ++st) {
                const f4 vf = *(const f4 *)(sV + (16 * c + 4 * lg + st) * 64 + 4 * sd_slot(16 * c + 4 * lg + st, li));
#pragma unroll
                for (int u = 0; u < 4; ++u) o[u] = mfma4(s[c][st], vf[u], o[u]);
            }
        __builtin_amdgcn_s_waitcnt(0x0f70);   // vmcnt(0): this wave's loads of the next K
        __syncthreads();
        __builtin_amdgcn_sched_barrier(0);
        if (more) issue(rv, sV, k0 + SD_T);
        __builtin_amdgcn_sched_barrier(0);
    }

    if (part_o) {   // a part of a split range: unnormalised rows and (max, sum)
        if (lg == 0 && my_q < Tq) {
            part_ml[(wave * 16 + li) * 2] = m_run;
            part_ml[(wave * 16 + li) * 2 + 1] = l_run;
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int row = wave * 16 + 4 * lg + r;
            f4 val = {o[0][r], o[1][r], o[2][r], o[3][r]};
            *(f4 *)(part_o + row * 64 + 4 * li) = val;
        }
        return;
    }
    // the row statistics a recomputing backward needs: (max, sum) of query my_q
    if (stats && lg == 0 && my_q < Tq) {
        float *st = stats + (((int64_t)b * Hq + h) * Tq + my_q) * 2;
        st[0] = m_run;
        st[1] = l_run;
    }
    // normalise by l of query qw + 4lg + r and store float4 along d
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const float lr = __shfl(l_run, 4 * lg + r, 64);
        const int qi = qw + 4 * lg + r;
        if (qi < Tq) {
            const float inv = 1.0f / lr;
            f4 val = {o[0][r] * inv, o[1][r] * inv, o[2][r] * inv, o[3][r] * inv};
            *(f4 *)(out + (merged ? ((int64_t)b * Tq + qi) * Hq + h : ((int64_t)b * Hq + h) * Tq + qi) * 64 +
                    4 * li) = val;
        }
    }
}

extern "C" __global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4, 4)))
sdpa_hd64(const float *__restrict__ q, const float *__restrict__ k, const float *__restrict__ v,
          const float *__restrict__ mask, float *__restrict__ out, int Hq, int Hkv, int Tq, int Tkv,
          float scale, int causal, int merged, float *__restrict__ stats, int64_t mask_bs) {
    // grid (Hq, B, query tiles), the last query tile first: under a causal
    // mask it has the most key tiles, and dispatching the heaviest workgroups
    // first keeps the chip busy to the end (longest-first order)
    sdpa_hd64_body(q, k, v, mask, out, Hq, Hkv, Tq, Tkv, scale, causal, merged, stats, blockIdx.x, blockIdx.y,
                   (gridDim.z - 1 - blockIdx.z) * 64, 0, (Tkv + SD_T - 1) / SD_T, nullptr, nullptr, mask_bs);
}

// The same over a work list, for grids too small to fill the chip (few (b, h)
// pairs, long rows): a query tile's key range is cut into parts of at most
// a fixed number of key blocks.  work[i] = (query tile, first key block, key
// blocks, slot): slot < 0 -- the tile's only part, stored as sdpa_hd64 does;
// otherwise the part's unnormalised rows go to part_o[bh][slot][64][64] and
// its (max, sum) to part_ml[bh][slot][64][2].  Workgroup x: work item x / BH,
// (b, h) pair x % BH, BH = B * Hq (the list is sorted longest part first).
extern "C" __global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4, 4)))
sdpa_hd64_split(const float *__restrict__ q, const float *__restrict__ k, const float *__restrict__ v,
                const float *__restrict__ mask, float *__restrict__ out, int Hq, int Hkv, int Tq, int Tkv,
                float scale, int causal, int merged, const int4 *__restrict__ work, int BH, int nslots,
                float *__restrict__ part_o, float *__restrict__ part_ml, int64_t mask_bs) {
    const int bh = blockIdx.x % BH;
    const int4 w = work[blockIdx.x / BH];
    const int h = bh % Hq, b = bh / Hq;
    float *po = w.w < 0 ? nullptr : part_o + ((int64_t)bh * nslots + w.w) * 64 * 64;
    float *pm = w.w < 0 ? nullptr : part_ml + ((int64_t)bh * nslots + w.w) * 64 * 2;
    sdpa_hd64_body(q, k, v, mask, out, Hq, Hkv, Tq, Tkv, scale, causal, merged, nullptr, h, b, w.x * 64, w.y,
                   w.y + w.z, po, pm, mask_bs);
}

// Merge of the parts of a split query tile: workgroup (tile x of the list
// tiles[], (b, h) pair y); thread = (query tid / 4, d = 16 (tid % 4) .. +15).
// m = max m_p, w_p = e^(m_p - m) (0 for a part whose keys were all masked),
// out = sum_p w_p o_p / sum_p w_p l_p.  A tile has at most SPLIT_MAXP parts;
// every part's loads are issued before the first use (clamped part index,
// weight 0 past the last part).
#define SPLIT_MAXP 8
extern "C" __global__ void __launch_bounds__(256)
sdpa_hd64_combine(const int2 *__restrict__ tiles, const float *__restrict__ part_o, const float *__restrict__ part_ml,
                  float *__restrict__ out, int Hq, int Tq, int merged, int nslots) {
    const int2 t = tiles[blockIdx.x];   // (query tile, first slot); parts = next entry's slot - this one's
    const int np = tiles[blockIdx.x + 1].y - t.y;
    const int bh = blockIdx.y, h = bh % Hq, b = bh / Hq;
    const int r = threadIdx.x >> 2, d0 = (threadIdx.x & 3) * 16;
    const int qi = t.x * 64 + r;
    if (qi >= Tq) return;
    const float *ml = part_ml + ((int64_t)bh * nslots + t.y) * 64 * 2 + r * 2;
    const float *po = part_o + ((int64_t)bh * nslots + t.y) * 64 * 64 + r * 64 + d0;
    float mp[SPLIT_MAXP], lp[SPLIT_MAXP];
    f4 op[SPLIT_MAXP][4];
#pragma unroll
    for (int p = 0; p < SPLIT_MAXP; ++p) {
        const int pc = min(p, np - 1);
        mp[p] = ml[(int64_t)pc * 64 * 2];
        lp[p] = ml[(int64_t)pc * 64 * 2 + 1];
#pragma unroll
        for (int u = 0; u < 4; ++u) op[p][u] = *(const f4 *)(po + (int64_t)pc * 64 * 64 + 4 * u);
    }
    float m = -INFINITY;
#pragma unroll
    for (int p = 0; p < SPLIT_MAXP; ++p)
        if (p < np) m = fmaxf(m, mp[p]);
    float l = 0.f;
    f4 acc[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) acc[u] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int p = 0; p < SPLIT_MAXP; ++p) {
        if (p >= np) continue;
        const float wp = mp[p] == -INFINITY ? 0.f : __expf(mp[p] - m);
        l += lp[p] * wp;
#pragma unroll
        for (int u = 0; u < 4; ++u) acc[u] += op[p][u] * wp;
    }
    const float inv = 1.0f / l;
    float *o = out + (merged ? ((int64_t)b * Tq + qi) * Hq + h : ((int64_t)b * Hq + h) * Tq + qi) * 64 + d0;
#pragma unroll
    for (int u = 0; u < 4; ++u) *(f4 *)(o + 4 * u) = acc[u] * inv;
}

// Generic SDPA for any hd <= 256: one wave per query row, online softmax in
// fp32, the lane dimension over hd.
extern "C" __global__ void __launch_bounds__(256)
sdpa_rows(const float *__restrict__ q, const float *__restrict__ k, const float *__restrict__ v,
          const float *__restrict__ mask, float *__restrict__ out, int B, int Hq, int Hkv, int Tq, int Tkv,
          int hd, float scale, int causal, int merged, int64_t mask_bs) {
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= (int64_t)B * Hq * Tq) return;
    const int tq = (int)(row % Tq);
    const int h = (int)((row / Tq) % Hq), b = (int)(row / ((int64_t)Tq * Hq));
    if (mask) mask += (int64_t)b * mask_bs;   // a board's own mask (mask_bs 0: one mask for all)
    const int kvh = h / (Hq / Hkv);
    const float *qr = q + row * hd;
    const float *kb = k + ((int64_t)b * Hkv + kvh) * Tkv * hd;
    const float *vb = v + ((int64_t)b * Hkv + kvh) * Tkv * hd;
    float qv[4], acc[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int d = lane + 64 * j;
        qv[j] = d < hd ? qr[d] : 0.f;
        acc[j] = 0.f;
    }
    float m = -INFINITY, l = 0.f;
    const int kend = causal ? min(Tkv, tq + 1 + (Tkv - Tq)) : Tkv;
    for (int tk = 0; tk < kend; ++tk) {
        const float *kr = kb + (int64_t)tk * hd;
        float dot = 0.f;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int d = lane + 64 * j;
            if (d < hd) dot += qv[j] * kr[d];
        }
        float x = wave_sum(dot) * scale;
        if (mask) x += mask[(int64_t)tq * Tkv + tk];
        const float m_new = fmaxf(m, x);
        if (m_new == -INFINITY) continue;
        const float alpha = __expf(m - m_new), p = __expf(x - m_new);
        l = l * alpha + p;
        const float *vr = vb + (int64_t)tk * hd;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int d = lane + 64 * j;
            acc[j] = acc[j] * alpha + (d < hd ? p * vr[d] : 0.f);
        }
        m = m_new;
    }
    float *o = out + (merged ? ((int64_t)b * Tq + tq) * Hq + h : row) * hd;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int d = lane + 64 * j;
        if (d < hd) o[d] = acc[j] / l;
    }
}

// ---------------------------------------------------------------- decode (KV cache)
// Decode attention, one query row per head over keys [0, *posp] of the cache,
// split over chunks of 64 keys.  A workgroup owns one kv head and one chunk
// and all rep = H / Hkv query heads of the group (rep <= 16).  K and V of the
// chunk are staged in LDS with coalesced float4 loads; wave w scores the
// chunk's 64 keys (lane = key) against queries w, w+4, ...; the chunk's
// (max, sum) per query come from wave reductions; o = sum p v with lane =
// dimension.  hd = 64.  part_o [H][gridDim.x][64], part_ml [H][gridDim.x][2];
// sdpa_decode_combine merges the chunks that hold keys.
#define DEC_CH 64
#define DEC_LD 68
extern "C" __global__ void __launch_bounds__(256)
sdpa_decode_partial(const float *__restrict__ q, const float *__restrict__ kc, const float *__restrict__ vc,
                    float *__restrict__ part_o, float *__restrict__ part_ml, int H, int Hkv,
                    const int *__restrict__ posp, int ld, float scale) {
    __shared__ __attribute__((aligned(16))) float sQ[16 * 64];
    __shared__ __attribute__((aligned(16))) float sK[DEC_CH * DEC_LD];
    __shared__ __attribute__((aligned(16))) float sV[DEC_CH * 64];
    __shared__ float sP[16 * DEC_CH];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int kvh = blockIdx.y, chunk = blockIdx.x, nchunk = gridDim.x;
    const int rep = H / Hkv, h0 = kvh * rep;
    const int Tkv = *posp + 1;
    const int k0 = chunk * DEC_CH;
    if (k0 >= Tkv) return;    // chunk past the current length (grid sized for n_ctx)
    const int nk = min(DEC_CH, Tkv - k0);
    // every load issued before the first LDS store, unconditionally (clamped
    // rows, zeroed afterwards): one memory round trip instead of one per row
    // group (a guarded load is a branch with a wait after it)
    const int nq = rep * 16;   // float4 of the group's queries (rep <= 16)
    const f4 qv = *(const f4 *)(q + (int64_t)h0 * 64 + 4 * min(tid, nq - 1));
    const float *kb = kc + ((int64_t)kvh * ld + k0) * 64, *vb = vc + ((int64_t)kvh * ld + k0) * 64;
    f4 kr[4], vr[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int f = tid + 256 * j, r = min(f >> 4, nk - 1), c = (f & 15) * 4;
        kr[j] = *(const f4 *)(kb + r * 64 + c);
        vr[j] = *(const f4 *)(vb + r * 64 + c);
    }
    __builtin_amdgcn_sched_barrier(0);
    if (tid < nq) *(f4 *)(sQ + 4 * tid) = qv;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int f = tid + 256 * j, r = f >> 4, c = (f & 15) * 4;
        const f4 z = {0.f, 0.f, 0.f, 0.f};
        *(f4 *)(sK + r * DEC_LD + c) = r < nk ? kr[j] : z;
        *(f4 *)(sV + r * 64 + c) = r < nk ? vr[j] : z;
    }
    __syncthreads();
    // scores: wave w, queries j = w, w+4, ... (lane = key)
    for (int j = wave; j < rep; j += 4) {
        float acc = 0.f;
#pragma unroll
        for (int c = 0; c < 16; ++c) {
            const f4 kv = *(const f4 *)(sK + lane * DEC_LD + 4 * c);
            const f4 qv = *(const f4 *)(sQ + j * 64 + 4 * c);
            acc += (qv[0] * kv[0] + qv[1] * kv[1]) + (qv[2] * kv[2] + qv[3] * kv[3]);
        }
        const float sc = lane < nk ? acc * scale : -INFINITY;
        float m = sc;
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
        const float p = lane < nk ? __expf(sc - m) : 0.f;
        float l = p;
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) l += __shfl_xor(l, o, 64);
        sP[j * DEC_CH + lane] = p;
        if (lane == 0) {
            part_ml[((int64_t)(h0 + j) * nchunk + chunk) * 2] = m;
            part_ml[((int64_t)(h0 + j) * nchunk + chunk) * 2 + 1] = l;
        }
    }
    __syncthreads();
    // o[j][d] = sum_key p[j][key] v[key][d]: wave w, queries w, w+4, ...; lane = d
    for (int j = wave; j < rep; j += 4) {
        // four independent chains (keys t = 4 i + u), added at the end
        float o4[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll 4
        for (int t = 0; t < DEC_CH; t += 4)
#pragma unroll
            for (int u = 0; u < 4; ++u) o4[u] += sP[j * DEC_CH + t + u] * sV[(t + u) * 64 + lane];
        part_o[((int64_t)(h0 + j) * nchunk + chunk) * 64 + lane] = (o4[0] + o4[1]) + (o4[2] + o4[3]);
    }
}

// out[h][d] = sum_c o_c[d] e^(m_c - m) / sum_c l_c e^(m_c - m); one wave per
// head: lanes load the chunks' (max, sum) pairs (64 at a time), the weights
// are broadcast back with shuffles while lane = d accumulates o.
extern "C" __global__ void __launch_bounds__(64)
sdpa_decode_combine(const float *__restrict__ part_o, const float *__restrict__ part_ml, float *__restrict__ out,
                    int stride, const int *__restrict__ posp) {
    const int h = blockIdx.x, lane = threadIdx.x;
    const int nchunk = (*posp + DEC_CH) / DEC_CH;
    const float *ml = part_ml + (int64_t)h * stride * 2, *po = part_o + (int64_t)h * stride * 64;
    if (nchunk <= 64) {
        // one round trip: every chunk's (max, sum) and output loaded before
        // the first use (clamped index, weight 0 past the last chunk); the
        // same operations in the same order as the loop below
        const int cl = min(lane, nchunk - 1);
        const float mc = ml[2 * cl], lcv = ml[2 * cl + 1];
        float pv[64];
#pragma unroll
        for (int t = 0; t < 64; ++t) pv[t] = po[(int64_t)min(t, nchunk - 1) * 64 + lane];
        float m = lane < nchunk ? mc : -INFINITY;
#pragma unroll
        for (int s = 32; s > 0; s >>= 1) m = fmaxf(m, __shfl_xor(m, s, 64));
        const float w = (lane < nchunk && mc != -INFINITY) ? __expf(mc - m) : 0.f;
        float l = lane < nchunk ? lcv * w : 0.f, o = 0.f;
#pragma unroll
        for (int t = 0; t < 64; ++t) o += pv[t] * __shfl(w, t, 64);
#pragma unroll
        for (int s = 32; s > 0; s >>= 1) l += __shfl_xor(l, s, 64);
        out[(int64_t)h * 64 + lane] = o / l;
        return;
    }
    float m = -INFINITY;
    for (int c = lane; c < nchunk; c += 64) m = fmaxf(m, ml[2 * c]);
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
    float l = 0.f, o = 0.f;
    for (int c0 = 0; c0 < nchunk; c0 += 64) {
        const int c = c0 + lane;
        float w = 0.f, lc = 0.f;
        if (c < nchunk) {
            const float mc = ml[2 * c];
            w = mc == -INFINITY ? 0.f : __expf(mc - m);
            lc = ml[2 * c + 1] * w;
        }
        l += lc;
        // loads of every chunk issued unconditionally (clamped index, weight 0
        // past the last chunk) so they overlap
#pragma unroll 16
        for (int t = 0; t < 64; ++t) {
            const float wt = __shfl(w, t, 64);
            o += po[(int64_t)min(c0 + t, nchunk - 1) * 64 + lane] * wt;
        }
    }
#pragma unroll
    for (int s = 32; s > 0; s >>= 1) l += __shfl_xor(l, s, 64);
    out[(int64_t)h * 64 + lane] = o / l;
}

// ---------------------------------------------------------------- decode GEMV
// y = W x for one input row, a wave per output row (RW rows per wave, 4
// waves), the input staged once per workgroup in LDS -- optionally RMS-
// normalised on the way (rmsnorm_fwd's arithmetic: fp64 sum of squares,
// s = (float)(1/sqrt(ms/K + 1e-6)), xn = (x*s)*nw).  Each wave issues the
// small loads and the input first, then its first PRE float4 per lane and
// row, so the normalisation and staging run while the weight stream is in
// flight.
//   mode 0: rows index the concatenation of up to three matrices; res (one
//           matrix) is added last.
//   mode 1: row n pairs W0 and W1: y0[n] = silu(W0 x + b0)[n] * (W1 x + b1)[n]
//           (the reference's silu_fwd + mul_fwd).
//   mode 2: q | k | v projections of one decode position with RoPE and the
//           cache append fused (hd = 64): a wave computes the rotation pair
//           (d, d + 32) of a q or k head, rotates it with the table row *posp
//           (kernels.c:249-264 arithmetic) and writes q to y0 [H][64], k to
//           kc[kvh][*posp], v rows (in pairs) to vc[kvh][*posp].
// K % 4 == 0, 16-byte aligned rows, K <= 8192.
struct DecGemvArgs {
    const float *x, *nw, *res;
    const float *W[3];
    const float *b[3];
    float *y[3];
    int N[3];
    int K, mode;
    const float *cos_t, *sin_t;
    const int *posp;
    float *kc, *vc;
    int ld;
};


// Member m of a 3-pointer argument array, by selects: indexing the array with
// a run-time m makes the compiler read the pointer from the argument block
// in memory, and that load queues behind the weight loads already in flight.
template <typename T>
__device__ __forceinline__ T sel3(const T (&a)[3], int m) {
    return m == 0 ? a[0] : (m == 1 ? a[1] : a[2]);
}

// row (in the concatenated row space) of the i-th dot product of this wave
__device__ __forceinline__ void dec_rows(const DecGemvArgs &p, int unit, int i, int &m, int &row) {
    if (p.mode == 2) {
        const int qk_pairs = (p.N[0] + p.N[1]) >> 1;
        if (unit < qk_pairs) {
            const int head = unit >> 5, d = unit & 31;
            row = head * 64 + d + 32 * i;          // within q | k
        } else {
            row = p.N[0] + p.N[1] + 2 * (unit - qk_pairs) + i;
        }
    } else if (p.mode == 1) {
        m = i;
        return;
    } else {
        row = unit;
    }
    m = 0;
    if (row >= p.N[0]) { row -= p.N[0]; m = 1; }
    if (m == 1 && row >= p.N[1]) { row -= p.N[1]; m = 2; }
}

template <int RW, int PRE, int DOTS, int XPT>
__device__ __forceinline__ void dec_gemv_body(const DecGemvArgs &p) {
#pragma clang fp contract(off)
    // the staged input: K <= 1024 XPT floats (LDS sized to it, so that short
    // rows do not reserve the 32 KB of the longest)
    __shared__ __attribute__((aligned(16))) float xs[1024 * XPT];
    __shared__ double red[4];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int K = p.K, K4 = K >> 2;
    // units: mode 0 rows, mode 1 row pairs (gate, up), mode 2 RoPE / v pairs
    const int units = p.mode == 0 ? p.N[0] + p.N[1] + p.N[2]
                      : p.mode == 1 ? p.N[0] : (p.N[0] + p.N[1] + p.N[2]) >> 1;
    const int u0 = (blockIdx.x * 4 + wave) * RW;
    const float *wr[RW][DOTS];
    int um[RW][DOTS], urow[RW][DOTS];
#pragma unroll
    for (int r = 0; r < RW; ++r)
#pragma unroll
        for (int i = 0; i < DOTS; ++i) {
            int m = 0, row = 0;
            dec_rows(p, min(u0 + r, units - 1), i, m, row);
            if (p.mode == 1) row = min(u0 + r, units - 1);
            um[r][i] = m;
            urow[r][i] = row;
            wr[r][i] = sel3(p.W, m) + (int64_t)row * K;
        }
    // Load order.  A wave's loads complete in issue order, so what is needed
    // first is issued first: the position, the epilogue's bias and residual
    // values and the input, then the weight rows (the bulk), then the RoPE
    // table values (their address needs the position).  The input is
    // normalised and staged while the weight rows stream in, and the
    // epilogue reads nothing from memory.
    // Every load is unconditional (a clamped index, or a valid stand-in for
    // an absent operand, with the value selected afterwards): a load under a
    // branch makes the compiler wait for all loads in flight where the
    // branches join, which would serialise the stream.
    const int *pp = p.mode == 2 ? p.posp : (const int *)p.x;
    const int pos = p.mode == 2 ? *pp : 0;
    float eb[RW][DOTS], er[RW];
    bool hb[RW][DOTS];
#pragma unroll
    for (int r = 0; r < RW; ++r) {
#pragma unroll
        for (int i = 0; i < DOTS; ++i) {
            const float *bm = sel3(p.b, um[r][i]);
            hb[r][i] = bm != nullptr;
            eb[r][i] = *(bm ? bm + urow[r][i] : p.x);
        }
        const bool hr = p.mode == 0 && p.res;
        er[r] = *(hr ? p.res + urow[r][0] : p.x);
    }
    // (raw values here; lanes past the row end hold a duplicate of its last
    // group and are zeroed where the values are used, after the waits)
    f4 xv4[XPT], nv4[XPT];
    const float *nwp = p.nw ? p.nw : p.x;
#pragma unroll
    for (int e = 0; e < XPT; ++e) {
        const int cc = min(tid + 256 * e, K4 - 1);
        xv4[e] = *(const f4 *)(p.x + 4 * cc);
        if (p.nw) nv4[e] = *(const f4 *)(nwp + 4 * cc);
    }
    __builtin_amdgcn_sched_barrier(0);   // keep the issue order: the small loads first
    f4 pw[RW][DOTS][PRE];
#pragma unroll
    for (int r = 0; r < RW; ++r)
#pragma unroll
        for (int i = 0; i < DOTS; ++i)
#pragma unroll
            for (int e = 0; e < PRE; ++e)
                pw[r][i][e] = __builtin_nontemporal_load((const f4 *)wr[r][i] + min(lane + 64 * e, K4 - 1));
    __builtin_amdgcn_sched_barrier(0);
    // RoPE: the rotation pair (d, d + 32) of a q or k head (d = row & 31).
    // Loaded unconditionally, from the input row when there is no table (a
    // branch around the loads makes the compiler wait for every load in
    // flight where the branches join).
    float rc0[RW], rs0[RW], rc1[RW], rs1[RW];
    {
        const bool rope = p.mode == 2;
        const float *co = rope ? p.cos_t + (int64_t)pos * 64 : p.x;
        const float *si = rope ? p.sin_t + (int64_t)pos * 64 : p.x;
#pragma unroll
        for (int r = 0; r < RW; ++r) {
            const int d = urow[r][0] & 31;
            const int d0 = rope ? d : min(d, K - 1), d1 = rope ? d + 32 : min(d + 32, K - 1);
            rc0[r] = co[d0];
            rs0[r] = si[d0];
            rc1[r] = co[d1];
            rs1[r] = si[d1];
        }
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int e = 0; e < XPT; ++e)
        if (tid + 256 * e >= K4) xv4[e] = f4{0.f, 0.f, 0.f, 0.f};
    if (p.nw) {
        double ss = 0.0;
#pragma unroll
        for (int e = 0; e < XPT; ++e)
#pragma unroll
            for (int i = 0; i < 4; ++i) ss += (double)xv4[e][i] * (double)xv4[e][i];
        ss = wave_sum_d(ss);
        if (lane == 0) red[wave] = ss;
        __syncthreads();
        const double ms = (((red[0] + red[1]) + red[2]) + red[3]) / K;
        const float s = (float)(1.0 / sqrt(ms + 1e-6));
#pragma unroll
        for (int e = 0; e < XPT; ++e)
#pragma unroll
            for (int i = 0; i < 4; ++i) xv4[e][i] = (xv4[e][i] * s) * nv4[e][i];
    }
#pragma unroll
    for (int e = 0; e < XPT; ++e) {
        const int c = tid + 256 * e;
        if (c < K4) *(f4 *)(xs + 4 * c) = xv4[e];
    }
    __syncthreads();
    float acc[RW][DOTS];
#pragma unroll
    for (int r = 0; r < RW; ++r)
#pragma unroll
        for (int i = 0; i < DOTS; ++i) acc[r][i] = 0.f;
#pragma unroll
    for (int e = 0; e < PRE; ++e) {
        const int c = lane + 64 * e;
        if (c < K4) {   // (lanes past the row end loaded a duplicate: skipped here)
            const f4 xv = *(const f4 *)(xs + 4 * c);
#pragma unroll
            for (int r = 0; r < RW; ++r)
#pragma unroll
                for (int i = 0; i < DOTS; ++i)
                    acc[r][i] += (pw[r][i][e].x * xv.x + pw[r][i][e].y * xv.y) +
                                 (pw[r][i][e].z * xv.z + pw[r][i][e].w * xv.w);
        }
    }
    for (int c = lane + 64 * PRE; c < K4; c += 64) {
        const f4 xv = *(const f4 *)(xs + 4 * c);
#pragma unroll
        for (int r = 0; r < RW; ++r)
#pragma unroll
            for (int i = 0; i < DOTS; ++i) {
                const f4 w = __builtin_nontemporal_load((const f4 *)wr[r][i] + c);
                acc[r][i] += (w.x * xv.x + w.y * xv.y) + (w.z * xv.z + w.w * xv.w);
            }
    }
#pragma unroll
    for (int r = 0; r < RW; ++r) {
        const float a0 = wave_sum(acc[r][0]);
        const float a1 = DOTS == 2 ? wave_sum(acc[r][DOTS - 1]) : 0.f;
        const int unit = u0 + r;
        if (lane != 0 || unit >= units) continue;
        if (p.mode == 0) {
            const int m = um[r][0], row = urow[r][0];
            float v = hb[r][0] ? a0 + eb[r][0] : a0;
            if (p.res) v = er[r] + v;
            sel3(p.y, m)[row] = v;
        } else if (p.mode == 1) {
            const float g = hb[r][0] ? a0 + eb[r][0] : a0;
            const float u = hb[r][DOTS - 1] ? a1 + eb[r][DOTS - 1] : a1;
            p.y[0][unit] = ncm_act(g, ACT_SILU) * u;
        } else {
            const int m0 = um[r][0], row0 = urow[r][0], row1 = urow[r][DOTS - 1];
            const float v0 = hb[r][0] ? a0 + eb[r][0] : a0;
            const float v1 = hb[r][DOTS - 1] ? a1 + eb[r][DOTS - 1] : a1;
            if (m0 == 2) {      // v rows: plain append
                p.vc[((int64_t)(row0 >> 6) * p.ld + pos) * 64 + (row0 & 63)] = v0;
                p.vc[((int64_t)(row1 >> 6) * p.ld + pos) * 64 + (row1 & 63)] = v1;
            } else {
                const int d = row0 & 63;          // 0..31; row1 = row0 + 32
                const float y0 = v0 * rc0[r] + (-v1) * rs0[r];
                const float y1 = v1 * rc1[r] + v0 * rs1[r];
                float *dst = m0 == 0 ? p.y[0] + (row0 & ~63)
                                     : p.kc + ((int64_t)(row0 >> 6) * p.ld + pos) * 64;
                dst[d] = y0;
                dst[d + 32] = y1;
            }
        }
    }
}

// d<DOTS>: dot products per unit (1 for mode 0, 2 for modes 1 and 2);
// x<XPT>: input float4 per thread (K <= 1024 XPT)
#define DEC_GEMV(name, RW, PRE, DOTS, XPT) \
    extern "C" __global__ void __launch_bounds__(256) name(DecGemvArgs p) { dec_gemv_body<RW, PRE, DOTS, XPT>(p); }
DEC_GEMV(dec_gemv_d1_r1_p4_x1, 1, 4, 1, 1)
DEC_GEMV(dec_gemv_d1_r4_p4_x1, 4, 4, 1, 1)
DEC_GEMV(dec_gemv_d1_r1_p20_x5, 1, 20, 1, 5)
DEC_GEMV(dec_gemv_d1_r1_p8_x8, 1, 8, 1, 8)
DEC_GEMV(dec_gemv_d2_r1_p4_x1, 1, 4, 2, 1)
DEC_GEMV(dec_gemv_d2_r2_p4_x1, 2, 4, 2, 1)
DEC_GEMV(dec_gemv_d2_r1_p8_x8, 1, 8, 2, 8)

// ---------------------------------------------------------------- decode GEMV, workgroup per row pair
// For the decode products with too few rows to give every CU a wave per row
// (the o-projection and the down projection: 896 rows of 896 or 4864), a
// workgroup owns R rows and its 256 threads split K: thread t holds float4
// t + 256 e of the input in registers and multiplies it with the same float4
// of each of its rows; the 256 partial dot products are added by a wave
// reduction and then, across the four waves in order, through LDS.  The
// input never goes through LDS, and all of a thread's loads are issued
// before the first wait (input, weight rows, then the epilogue's bias and
// residual).  y[n] = res[n] + (W x)[n] (+ bias), dec_gemv's mode 0 over one
// matrix.  K % 4 == 0, K <= 1024 XPT.  (A wave per row, as dec_gemv_body
// streams it, leaves a quarter of the CUs idle at 896 rows.)
template <int R, int XPT>
__device__ __forceinline__ void dec_wg_body(const DecGemvArgs &p) {
#pragma clang fp contract(off)
    __shared__ float red[4][R];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int K = p.K, K4 = K >> 2, N = p.N[0];
    const int n0 = blockIdx.x * R;
    f4 xv[XPT];
#pragma unroll
    for (int e = 0; e < XPT; ++e) xv[e] = *(const f4 *)(p.x + 4 * min(tid + 256 * e, K4 - 1));
    __builtin_amdgcn_sched_barrier(0);
    f4 w[R][XPT];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int e = 0; e < XPT; ++e)
            w[r][e] = __builtin_nontemporal_load((const f4 *)(p.W[0] + (int64_t)min(n0 + r, N - 1) * K) +
                                                 min(tid + 256 * e, K4 - 1));
    __builtin_amdgcn_sched_barrier(0);
    // the epilogue's values (used by threads r < R; a stand-in address when absent)
    const int nr = min(n0 + min(tid, R - 1), N - 1);
    const float eb = *(p.b[0] ? p.b[0] + nr : p.x), er = *(p.res ? p.res + nr : p.x);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int e = 0; e < XPT; ++e)
        if (tid + 256 * e >= K4) xv[e] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int r = 0; r < R; ++r) {
        float a = 0.f;
#pragma unroll
        for (int e = 0; e < XPT; ++e)
            a += (w[r][e].x * xv[e].x + w[r][e].y * xv[e].y) + (w[r][e].z * xv[e].z + w[r][e].w * xv[e].w);
        a = wave_sum(a);
        if (lane == 0) red[wave][r] = a;
    }
    __syncthreads();
    if (tid >= R || n0 + tid >= N) return;
    float v = ((red[0][tid] + red[1][tid]) + red[2][tid]) + red[3][tid];
    if (p.b[0]) v += eb;
    if (p.res) v = er + v;
    p.y[0][n0 + tid] = v;
}

// r<R> rows per workgroup, x<XPT> input float4 per thread (K <= 1024 XPT)
#define DEC_WG(name, R, XPT) \
    extern "C" __global__ void __launch_bounds__(256) name(DecGemvArgs p) { dec_wg_body<R, XPT>(p); }
DEC_WG(dec_wg_plain_r2_x1, 2, 1)   // o-projection + residual (K <= 1024)
DEC_WG(dec_wg_plain_r2_x5, 2, 5)   // down projection + residual (K <= 5120)

// Position-driven pieces of a decode step, so that the step's launches do
// not change from one token to the next (it can be replayed as one graph):
// the token id is ids[*pos]; dec_argmax_part_k + dec_argmax_final_k write
// the greedy id of the logits to ids[*pos + 1] (argmax_rows_k's rule) and
// advance *pos.
extern "C" __global__ void __launch_bounds__(256)
dec_embed_k(const float *__restrict__ W, const int *__restrict__ ids, const int *__restrict__ pos,
            float *__restrict__ x, int D, int V) {
    int id = ids[*pos];
    if ((unsigned)id >= (unsigned)V) id = 0;
    for (int d = blockIdx.x * 256 + threadIdx.x; d < D; d += gridDim.x * 256) x[d] = W[(int64_t)id * D + d];
}

// LM head of a decode step, y = W . RMSNorm(x) over V rows (K <= 1024,
// K % 4 == 0, 16-byte aligned rows), as a grid-stride stream: a workgroup
// stages the normalised input once (dec_gemv_body's arithmetic), and each
// wave walks its groups of HEAD_RW rows (group g: rows (gw + g * waves) *
// HEAD_RW ..) with the next group's loads in flight while the current group is
// reduced.  Each wave also keeps the first maximum of its rows (it visits them
// in increasing order; strict '>'); the workgroup merges its four (ties to
// the lower index) into pv / pi [gridDim.x] for dec_argmax_final_k -- the
// first stage of the greedy argmax, fused.
#define HEAD_RW 4
extern "C" __global__ void __launch_bounds__(256)
dec_head_stream(const float *__restrict__ x, const float *__restrict__ nw, const float *__restrict__ W,
                float *__restrict__ y, int V, int K, float *__restrict__ pv, int *__restrict__ pi) {
#pragma clang fp contract(off)
    __shared__ __attribute__((aligned(16))) float xs[1024];
    __shared__ double red[4];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, K4 = K >> 2;
    const int gw = blockIdx.x * 4 + wave, NW = gridDim.x * 4;
    auto fetch = [&](f4 (&w)[HEAD_RW][4], int g) {
        const int r0 = (gw + g * NW) * HEAD_RW;
#pragma unroll
        for (int k = 0; k < HEAD_RW; ++k) {
            const f4 *row = (const f4 *)(W + (int64_t)min(r0 + k, V - 1) * K);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int c = lane + 64 * e;
                w[k][e] = c < K4 ? __builtin_nontemporal_load(row + c) : f4{0.f, 0.f, 0.f, 0.f};
            }
        }
    };
    f4 cur[HEAD_RW][4], nxt[HEAD_RW][4];
    fetch(cur, 0);
    // input: one float4 per thread (K <= 1024), RMSNorm as dec_gemv_body
    const f4 xv = tid < K4 ? *(const f4 *)(x + 4 * tid) : f4{0.f, 0.f, 0.f, 0.f};
    const f4 nv = tid < K4 ? *(const f4 *)(nw + 4 * tid) : f4{1.f, 1.f, 1.f, 1.f};
    double ss = 0.0;
#pragma unroll
    for (int i = 0; i < 4; ++i) ss += (double)xv[i] * (double)xv[i];
    ss = wave_sum_d(ss);
    if (lane == 0) red[wave] = ss;
    __syncthreads();
    const double ms = (((red[0] + red[1]) + red[2]) + red[3]) / K;
    const float sc = (float)(1.0 / sqrt(ms + 1e-6));
    if (tid < K4) {
        f4 v;
#pragma unroll
        for (int i = 0; i < 4; ++i) v[i] = (xv[i] * sc) * nv[i];
        *(f4 *)(xs + 4 * tid) = v;
    }
    __syncthreads();
    float best = -INFINITY;
    int bidx = 0x7fffffff;
    for (int g = 0;; ++g) {
        const int r0 = (gw + g * NW) * HEAD_RW;
        if (r0 >= V) break;
        fetch(nxt, g + 1);
#pragma unroll
        for (int k = 0; k < HEAD_RW; ++k) {
            float acc = 0.f;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int c = lane + 64 * e;
                if (c < K4) {
                    const f4 xq = *(const f4 *)(xs + 4 * c);
                    acc += (cur[k][e].x * xq.x + cur[k][e].y * xq.y) + (cur[k][e].z * xq.z + cur[k][e].w * xq.w);
                }
            }
            const float v = wave_sum(acc);
            const int row = r0 + k;
            if (row < V) {
                if (v > best) { best = v; bidx = row; }
                if (lane == 0) y[row] = v;
            }
        }
#pragma unroll
        for (int k = 0; k < HEAD_RW; ++k)
#pragma unroll
            for (int e = 0; e < 4; ++e) cur[k][e] = nxt[k][e];
    }
    __shared__ float wv[4];
    __shared__ int wi[4];
    if (lane == 0) {
        wv[wave] = best;
        wi[wave] = bidx;
    }
    __syncthreads();
    if (tid == 0) {
        float b = wv[0];
        int i = wi[0];
        for (int w = 1; w < 4; ++w)
            if (wv[w] > b || (wv[w] == b && wi[w] < i)) { b = wv[w]; i = wi[w]; }
        pv[blockIdx.x] = b;
        pi[blockIdx.x] = i;
    }
}

#define AMAX_PER 4096
// Stage 1: per block of AMAX_PER logits the first maximal value and its index
// (strict '>' scan per thread, ties to the lower index when merging).
extern "C" __global__ void __launch_bounds__(256)
dec_argmax_part_k(const float *__restrict__ x, int n, float *__restrict__ pv, int *__restrict__ pi) {
    __shared__ float bv[4];
    __shared__ int bi[4];
    const int tid = threadIdx.x, base = blockIdx.x * AMAX_PER;
    float best = -INFINITY;
    int bidx = 0x7fffffff;
#pragma unroll 16
    for (int j = 0; j < AMAX_PER / 256; ++j) {
        const int k = base + j * 256 + tid;
        const float v = k < n ? x[k] : -INFINITY;
        if (v > best) { best = v; bidx = k; }
    }
    for (int o = 32; o > 0; o >>= 1) {
        const float ov = __shfl_xor(best, o, 64);
        const int oi = __shfl_xor(bidx, o, 64);
        if (ov > best || (ov == best && oi < bidx)) { best = ov; bidx = oi; }
    }
    if ((tid & 63) == 0) { bv[tid >> 6] = best; bi[tid >> 6] = bidx; }
    __syncthreads();
    if (tid == 0) {
        float b = bv[0];
        int i = bi[0];
        for (int w = 1; w < 4; ++w)
            if (bv[w] > b || (bv[w] == b && bi[w] < i)) { b = bv[w]; i = bi[w]; }
        pv[blockIdx.x] = b;
        pi[blockIdx.x] = i;
    }
}

// Stage 2: merge the blocks, apply the reference's rule (index 0 when x[0]
// is NaN or nothing exceeds x[0] = -inf), write ids[*pos + 1], advance *pos.
extern "C" __global__ void __launch_bounds__(64)
dec_argmax_final_k(const float *__restrict__ x, const float *__restrict__ pv, const int *__restrict__ pi,
                   int nblk, int *__restrict__ ids, int *__restrict__ pos) {
    const int lane = threadIdx.x;
    float best = -INFINITY;
    int bidx = 0x7fffffff;
    for (int j = lane; j < nblk; j += 64) {
        const float v = pv[j];
        const int i = pi[j];
        if (v > best || (v == best && i < bidx)) { best = v; bidx = i; }
    }
    for (int o = 32; o > 0; o >>= 1) {
        const float ov = __shfl_xor(best, o, 64);
        const int oi = __shfl_xor(bidx, o, 64);
        if (ov > best || (ov == best && oi < bidx)) { best = ov; bidx = oi; }
    }
    if (lane == 0) {
        int i = bidx;
        if (x[0] != x[0] || i == 0x7fffffff) i = 0;
        const int p = *pos;
        ids[p + 1] = i;
        *pos = p + 1;
    }
}
