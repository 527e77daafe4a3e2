// ops.hip -- row-wise and elementwise kernels around the GEMMs.
#include "ncm_dev.h"

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
//     4 silu, 5 gelu, 6 gelu_tanh   (kernels.c:167-226, 829-874)
extern "C" __global__ void __launch_bounds__(256)
eltwise_k(const float *a, const float *b, float *y, float s, int64_t n, int op) {
#pragma clang fp contract(off)
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    const float v = a[i];
    switch (op) {
    case 0: y[i] = v + b[i]; break;
    case 1: y[i] = v * b[i]; break;
    case 2: y[i] = v * s; break;
    case 3: y[i] = y[i] + v; break;
    case 4: y[i] = ncm_act(v, ACT_SILU); break;
    case 5: y[i] = ncm_act(v, ACT_GELU); break;
    default: y[i] = ncm_act(v, ACT_GELU_TANH); break;
    }
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
#define SD_LD (64 + 8)

extern "C" __global__ void __launch_bounds__(256)
sdpa_hd64(const float *__restrict__ q, const float *__restrict__ k, const float *__restrict__ v,
          const float *__restrict__ mask, float *__restrict__ out, int Hq, int Hkv, int Tq, int Tkv,
          float scale, int causal) {
    __shared__ __attribute__((aligned(16))) float sK[SD_T * SD_LD];
    __shared__ __attribute__((aligned(16))) float sV[SD_T * SD_LD];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int li = lane & 15, lg = lane >> 4;
    const int h = blockIdx.y, b = blockIdx.z;
    const int kvh = h / (Hq / Hkv);
    const int q0 = blockIdx.x * 64, qw = q0 + wave * 16;
    const float *qb = q + ((int64_t)b * Hq + h) * Tq * 64;
    const float *kb = k + ((int64_t)b * Hkv + kvh) * Tkv * 64;
    const float *vb = v + ((int64_t)b * Hkv + kvh) * Tkv * 64;

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
    for (int k0 = 0; k0 < kend; k0 += SD_T) {
        __syncthreads();
        // stage K and V tiles (64 keys x 64 d), rows beyond Tkv as zero
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int f = tid + j * 256;
            const int r = f >> 4, c = (f & 15) * 4;
            const int key = k0 + r;
            f4 kv = {0.f, 0.f, 0.f, 0.f}, vv = {0.f, 0.f, 0.f, 0.f};
            if (key < Tkv) {
                kv = *(const f4 *)(kb + (int64_t)key * 64 + c);
                vv = *(const f4 *)(vb + (int64_t)key * 64 + c);
            }
            *(f4 *)(sK + r * SD_LD + c) = kv;
            *(f4 *)(sV + r * SD_LD + c) = vv;
        }
        __syncthreads();

        // S^T[c]: keys k0 + 16c + 4lg + r, query my_q
        f4 s[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            s[c] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int kc = 0; kc < 4; ++kc) {
                const f4 kf = *(const f4 *)(sK + (16 * c + li) * SD_LD + kc * 16 + 4 * lg);
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
                const f4 vf = *(const f4 *)(sV + (16 * c + 4 * lg + st) * SD_LD + 4 * li);
#pragma unroll
                for (int u = 0; u < 4; ++u) o[u] = mfma4(s[c][st], vf[u], o[u]);
            }
    }

    // normalise by l of query qw + 4lg + r and store float4 along d
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const float lr = __shfl(l_run, 4 * lg + r, 64);
        const int qi = qw + 4 * lg + r;
        if (qi < Tq) {
            const float inv = 1.0f / lr;
            f4 val = {o[0][r] * inv, o[1][r] * inv, o[2][r] * inv, o[3][r] * inv};
            *(f4 *)(out + (((int64_t)b * Hq + h) * Tq + qi) * 64 + 4 * li) = val;
        }
    }
}

// Generic SDPA for any hd <= 256: one wave per query row, online softmax in
// fp32, the lane dimension over hd.
extern "C" __global__ void __launch_bounds__(256)
sdpa_rows(const float *__restrict__ q, const float *__restrict__ k, const float *__restrict__ v,
          const float *__restrict__ mask, float *__restrict__ out, int B, int Hq, int Hkv, int Tq, int Tkv,
          int hd, float scale, int causal) {
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= (int64_t)B * Hq * Tq) return;
    const int tq = (int)(row % Tq);
    const int h = (int)((row / Tq) % Hq), b = (int)(row / ((int64_t)Tq * Hq));
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
    float *o = out + row * hd;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int d = lane + 64 * j;
        if (d < hd) o[d] = acc[j] / l;
    }
}

// ---------------------------------------------------------------- decode (KV cache)
// One decode position `pos`: RoPE (kernels.c:249-264 arithmetic, table row
// pos) on q [H][hd] and k [Hkv][hd] (the rows of the q/k projections), q
// written to qo [H][hd], k and v appended to the caches [Hkv][ld][hd] at
// row pos.  One thread per (head slot, d < hd/2) over H + Hkv slots, plus
// the v copy.
extern "C" __global__ void __launch_bounds__(256)
rope_append_k(const float *__restrict__ q, const float *__restrict__ k, const float *__restrict__ v,
              const float *__restrict__ cos_t, const float *__restrict__ sin_t, float *__restrict__ qo,
              float *__restrict__ kc, float *__restrict__ vc, int H, int Hkv, int hd, int ld, int pos) {
#pragma clang fp contract(off)
    const int h2 = hd >> 1;
    const int i = blockIdx.x * 256 + threadIdx.x;
    const int nrot = (H + Hkv) * h2;
    if (i < nrot) {
        const int slot = i / h2, d = i - slot * h2;
        const float *src = slot < H ? q + slot * hd : k + (slot - H) * hd;
        float *dst = slot < H ? qo + slot * hd : kc + ((int64_t)(slot - H) * ld + pos) * hd;
        const float *co = cos_t + (int64_t)pos * hd, *si = sin_t + (int64_t)pos * hd;
        const float a = src[d], b = src[d + h2];
        dst[d] = a * co[d] + (-b) * si[d];
        dst[d + h2] = b * co[d + h2] + a * si[d + h2];
    } else if (i < nrot + Hkv * hd) {
        const int j = i - nrot, kvh = j / hd, d = j - kvh * hd;
        vc[((int64_t)kvh * ld + pos) * hd + d] = v[j];
    }
}

// Decode attention, one query row per head over keys [0, Tkv) of the cache:
// split over key chunks of 256.  A workgroup owns one kv head and one chunk
// and all rep = H / Hkv query heads of the group (rep <= 16): thread t
// scores key c*256 + t against every query of the group, the chunk's
// (max, sum) per query come from block reductions, and o = sum p v with
// threads (g, d) = 4 key quarters x 64 dims, reduced through LDS.  hd = 64.
// part_o [H][nchunk][64], part_ml [H][nchunk][2]; sdpa_decode_combine
// merges the chunks.
#define DEC_CH 256
extern "C" __global__ void __launch_bounds__(256)
sdpa_decode_partial(const float *__restrict__ q, const float *__restrict__ kc, const float *__restrict__ vc,
                    float *__restrict__ part_o, float *__restrict__ part_ml, int H, int Hkv, int Tkv, int ld,
                    float scale) {
    __shared__ __attribute__((aligned(16))) float sQ[16 * 64];
    __shared__ float sP[16 * DEC_CH];
    __shared__ float sRed[16 * 4];
    __shared__ float sM[16], sL[16];
    __shared__ __attribute__((aligned(16))) float sO[4 * 16 * 64];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int kvh = blockIdx.y, chunk = blockIdx.x, nchunk = gridDim.x;
    const int rep = H / Hkv, h0 = kvh * rep;
    const int key = chunk * DEC_CH + tid;
    for (int i = tid; i < rep * 64; i += 256) sQ[i] = q[(int64_t)h0 * 64 + i];
    __syncthreads();
    float s[16];
    if (key < Tkv) {
        const float *kr = kc + ((int64_t)kvh * ld + key) * 64;
        f4 kv[16];
#pragma unroll
        for (int c = 0; c < 16; ++c) kv[c] = *(const f4 *)(kr + 4 * c);
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            if (j < rep) {
                float acc = 0.f;
#pragma unroll
                for (int c = 0; c < 16; ++c) {
                    const f4 qv = *(const f4 *)(sQ + j * 64 + 4 * c);
                    acc += qv[0] * kv[c][0] + qv[1] * kv[c][1] + qv[2] * kv[c][2] + qv[3] * kv[c][3];
                }
                s[j] = acc * scale;
            }
        }
    } else {
#pragma unroll
        for (int j = 0; j < 16; ++j) s[j] = -INFINITY;
    }
    // per-query chunk max
#pragma unroll
    for (int j = 0; j < 16; ++j) {
        if (j < rep) {
            float m = s[j];
#pragma unroll
            for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
            if (lane == 0) sRed[j * 4 + wave] = m;
        }
    }
    __syncthreads();
    if (tid < rep) sM[tid] = fmaxf(fmaxf(sRed[tid * 4], sRed[tid * 4 + 1]), fmaxf(sRed[tid * 4 + 2], sRed[tid * 4 + 3]));
    __syncthreads();
#pragma unroll
    for (int j = 0; j < 16; ++j) {
        if (j < rep) {
            const float m = sM[j];
            const float p = (m == -INFINITY || key >= Tkv) ? 0.f : __expf(s[j] - m);
            sP[j * DEC_CH + tid] = p;
            float l = p;
#pragma unroll
            for (int o = 32; o > 0; o >>= 1) l += __shfl_xor(l, o, 64);
            if (lane == 0) sRed[j * 4 + wave] = l;
        }
    }
    __syncthreads();
    if (tid < rep) sL[tid] = (sRed[tid * 4] + sRed[tid * 4 + 1]) + (sRed[tid * 4 + 2] + sRed[tid * 4 + 3]);
    // o partial: wave g sums keys 64g .. 64g+63 for every query, lane = d
    float acc[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) acc[j] = 0.f;
    const int kbase = chunk * DEC_CH + wave * 64;
    const int kn = min(64, Tkv - kbase);
    for (int t = 0; t < kn; ++t) {
        const float vv = vc[((int64_t)kvh * ld + kbase + t) * 64 + lane];
#pragma unroll
        for (int j = 0; j < 16; ++j)
            if (j < rep) acc[j] += sP[j * DEC_CH + wave * 64 + t] * vv;
    }
#pragma unroll
    for (int j = 0; j < 16; ++j)
        if (j < rep) sO[(wave * 16 + j) * 64 + lane] = acc[j];
    __syncthreads();
    for (int i = tid; i < rep * 64; i += 256) {
        const int j = i >> 6, d = i & 63;
        const float o = (sO[(0 * 16 + j) * 64 + d] + sO[(1 * 16 + j) * 64 + d]) +
                        (sO[(2 * 16 + j) * 64 + d] + sO[(3 * 16 + j) * 64 + d]);
        part_o[((int64_t)(h0 + j) * nchunk + chunk) * 64 + d] = o;
    }
    if (tid < rep) {
        part_ml[((int64_t)(h0 + tid) * nchunk + chunk) * 2] = sM[tid];
        part_ml[((int64_t)(h0 + tid) * nchunk + chunk) * 2 + 1] = sL[tid];
    }
}

// out[h][d] = sum_c o_c[d] e^(m_c - m) / sum_c l_c e^(m_c - m); one wave per head.
extern "C" __global__ void __launch_bounds__(64)
sdpa_decode_combine(const float *__restrict__ part_o, const float *__restrict__ part_ml, float *__restrict__ out,
                    int nchunk) {
    const int h = blockIdx.x, d = threadIdx.x;
    float m = -INFINITY;
    for (int c = 0; c < nchunk; ++c) m = fmaxf(m, part_ml[((int64_t)h * nchunk + c) * 2]);
    float l = 0.f, o = 0.f;
    for (int c = 0; c < nchunk; ++c) {
        const float mc = part_ml[((int64_t)h * nchunk + c) * 2];
        const float w = mc == -INFINITY ? 0.f : __expf(mc - m);
        l += part_ml[((int64_t)h * nchunk + c) * 2 + 1] * w;
        o += part_o[((int64_t)h * nchunk + c) * 64 + d] * w;
    }
    out[(int64_t)h * 64 + d] = o / l;
}
