// sample.hip -- temperature / top-k / nucleus sampling of one logits row on
// the device: the arithmetic of the reference's host sample_topkp
// (src/kernels.c:782-825), which copies the row to the host and qsorts all V
// entries per step (qwen.c:220-223, gpt2.c:194).
//
// Reference steps, with w_i = logits_i / temp (float) and ord the indices
// sorted by w descending (glibc's merge-sort qsort: equal values keep
// ascending index order):
//   keep = top_k > 0 ? min(top_k, V) : V
//   p_r = exp((double) w_ord[r] - w_ord[0]), den = serial sum, q_r = p_r / den
//   nkeep = first r with (q_0 + .. + q_{r-1}) - q_r > top_p, else keep
//   u = U * (q_0 + .. + q_{nkeep-1}),  U = (xorshift64*(rng) >> 11) * 2^-53
//   pick = ord[first r < nkeep with u <= q_0 + .. + q_r], else ord[nkeep-1]
//
// Device plan: a stable LSD radix sort of (order key, index) over 4 passes of
// 8 bits (smp_hist, smp_scatter per pass), fp64 probabilities with fixed-
// order block sums (smp_probs), and one workgroup (smp_finish) that locates
// the nucleus cut and the draw: a prefilter over block prefix sums, then an
// element scan inside the block.
//
// Certification: the device exp (ROCm device library) and glibc's exp may
// differ in the last bits, and the prefix sums are formed in another order
// than the reference's serial loop.  Every compared quantity (normalised
// prefix sums, at most ~1) is within eta = 8 * 2^-50 + 4 (n + 64) 2^-53 of
// its exact value on both sides (exp error plus gamma_n for any summation
// order of n non-negative terms), so a decision whose margin exceeds the
// combined bound is the reference's decision.  The kernel reports in *flag:
// 0 the id is certified equal to the reference's; 1 the draw fell within
// the bound of a boundary (an event of probability ~1e-10 per draw); 2 the
// row holds a non-finite w (outside the reference's defined behaviour).
#include "ncm_dev.h"

#define SMP_NT 1024     // threads of a sort block
#define SMP_SB 8192     // elements per sort block (SMP_NT threads x 8 rounds)
#define SMP_MAXB 32     // sort blocks -> V <= 262144
#define SMP_PB 1024     // elements per probability block (= finish workgroup)

// Order key of w: ascending key order = descending w.  -0 and +0 are one
// value (the reference's comparator finds them equal).
__device__ __forceinline__ unsigned smp_key(float w) {
    unsigned b = __float_as_uint(w);
    if ((b << 1) == 0u) b = 0u;
    const unsigned asc = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
    return ~asc;
}

// Digit histogram of radix pass `pass` for one sort block:
// hist[pass][d][block].  Pass 0 reads the logits (kin == null) and records
// a block's non-finite w in bad[block]; later passes read the previous
// pass's output.
extern "C" __global__ void __launch_bounds__(SMP_NT)
smp_hist(const float *__restrict__ x, float temp, const unsigned *__restrict__ kin, int n, int pass,
         int *__restrict__ hist, int nblk, int *__restrict__ bad) {
    __shared__ int cnt[256];
    __shared__ int anybad;
    const int tid = threadIdx.x, b = blockIdx.x, shift = 8 * pass;
    if (tid < 256) cnt[tid] = 0;
    if (tid == 0) anybad = 0;
    __syncthreads();
    int nf = 0;
#pragma unroll
    for (int r = 0; r < SMP_SB / SMP_NT; ++r) {
        const int e = b * SMP_SB + r * SMP_NT + tid;
        if (e < n) {
            unsigned k;
            if (kin) {
                k = kin[e];
            } else {
                const float w = x[e] / temp;
                nf |= !isfinite(w);
                k = smp_key(w);
            }
            atomicAdd(&cnt[(k >> shift) & 255u], 1);
        }
    }
    if (nf) anybad = 1;
    __syncthreads();
    if (tid < 256) hist[(pass * 256 + tid) * nblk + b] = cnt[tid];
    if (!kin && tid == 0) bad[b] = anybad;
}

// Stable scatter of one sort block by the digit of radix pass `pass`.
//   1. Wave w owns the block's elements [w * 512, (w + 1) * 512) in rounds
//      of 64: a lane's rank among its wave's earlier elements of the same
//      digit comes from ballots (lanes of the round with that digit) and a
//      wave-private running count per digit (no barrier).
//   2. Threads 0..255 (one per digit) scan the counts: the block's local
//      start of each digit, each wave's start inside it, and the digit's
//      global start from the pass's histogram (all blocks' counts of the
//      digit before this block, plus every count of smaller digits).
//   3. The elements are placed in LDS in sorted order and each digit's run
//      is written to global memory by consecutive threads (coalesced).
// Pass 0 forms (key, index) from the logits (kin == null).  A position
// outside [0, n) is never written (it cannot occur: the offsets come from
// the same elements).
#define SMP_W (SMP_NT / 64)
#define SMP_R (SMP_SB / SMP_NT)   // rounds per wave
extern "C" __global__ void __launch_bounds__(SMP_NT)
smp_scatter(const float *__restrict__ x, float temp, const unsigned *__restrict__ kin,
            const int *__restrict__ iin, int n, int pass, const int *__restrict__ hist, int nblk,
            unsigned *__restrict__ kout, int *__restrict__ iout) {
    __shared__ int gofs[256];          // global position minus local position, per digit
    __shared__ int wrun[SMP_W][256];   // per wave: digit counts, then the wave's local start
    __shared__ int wsg[4], wsl[4];     // digit-scan totals of the 4 digit waves (global, local)
    __shared__ unsigned sk[SMP_SB];
    __shared__ int si[SMP_SB];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, b = blockIdx.x, shift = 8 * pass;
    const int e0 = b * SMP_SB + wave * (SMP_R * 64) + lane;   // element of round r: e0 + 64 r
    const int nloc = min(SMP_SB, n - b * SMP_SB);
    unsigned kk[SMP_R];
    int ii[SMP_R], rk[SMP_R];
#pragma unroll
    for (int r = 0; r < SMP_R; ++r) {
        const int e = e0 + 64 * r;
        kk[r] = 0u;
        ii[r] = 0;
        if (e < n) {
            if (kin) {
                kk[r] = kin[e];
                ii[r] = iin[e];
            } else {
                kk[r] = smp_key(x[e] / temp);
                ii[r] = e;
            }
        }
    }
    // global start of the digit, less the wave-total part (threads 0..255;
    // the nblk <= 32 counts of a digit load together)
    int gpart = 0;
    if (tid < 256) {
        const int *hd = hist + (pass * 256 + tid) * nblk;
        int v[SMP_MAXB];
#pragma unroll
        for (int j = 0; j < SMP_MAXB; ++j) v[j] = j < nblk ? hd[j] : 0;
        int tot = 0, pre = 0;
#pragma unroll
        for (int j = 0; j < SMP_MAXB; ++j) {
            tot += v[j];
            pre += j < b ? v[j] : 0;
        }
        int incl = tot;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const int t = __shfl_up(incl, o, 64);
            if (lane >= o) incl += t;
        }
        if (lane == 63) wsg[wave] = incl;
        gpart = incl - tot + pre;
    }
    // 1. wave-local ranks (the wave's own row of wrun; one wave's LDS accesses are ordered)
#pragma unroll
    for (int j = 0; j < 4; ++j) wrun[wave][lane + 64 * j] = 0;
    const unsigned long long below = (1ull << lane) - 1ull;
#pragma unroll
    for (int r = 0; r < SMP_R; ++r) {
        const bool valid = e0 + 64 * r < n;
        const unsigned d = (kk[r] >> shift) & 255u;
        unsigned long long peers = __ballot(valid);
#pragma unroll
        for (int bit = 0; bit < 8; ++bit) {
            const bool on = (d >> bit) & 1u;
            const unsigned long long m = __ballot(on);
            peers &= on ? m : ~m;
        }
        const int before = wrun[wave][d];
        rk[r] = before + __popcll(peers & below);
        if (valid && (peers & below) == 0ull) wrun[wave][d] = before + __popcll(peers);
    }
    __syncthreads();
    // 2. per digit: block count, local start, global start, waves' starts
    int cnt = 0, incl = 0;
    if (tid < 256) {
#pragma unroll
        for (int w = 0; w < SMP_W; ++w) cnt += wrun[w][tid];
        incl = cnt;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const int t = __shfl_up(incl, o, 64);
            if (lane >= o) incl += t;
        }
        if (lane == 63) wsl[wave] = incl;
    }
    __syncthreads();
    if (tid < 256) {
        int pg = 0, pl = 0;
        for (int w = 0; w < wave; ++w) {
            pg += wsg[w];
            pl += wsl[w];
        }
        const int lstart = incl - cnt + pl;
        gofs[tid] = gpart + pg - lstart;
        int acc = lstart;
#pragma unroll
        for (int w = 0; w < SMP_W; ++w) {
            const int c = wrun[w][tid];
            wrun[w][tid] = acc;
            acc += c;
        }
    }
    __syncthreads();
    // 3. sorted order in LDS, then coalesced runs to global memory
#pragma unroll
    for (int r = 0; r < SMP_R; ++r) {
        if (e0 + 64 * r < n) {
            const int lp = wrun[wave][(kk[r] >> shift) & 255u] + rk[r];
            if ((unsigned)lp < (unsigned)SMP_SB) {
                sk[lp] = kk[r];
                si[lp] = ii[r];
            }
        }
    }
    __syncthreads();
    for (int lp = tid; lp < nloc; lp += SMP_NT) {
        const unsigned k = sk[lp];
        const int pos = gofs[(k >> shift) & 255u] + lp;
        if ((unsigned)pos < (unsigned)n) {
            kout[pos] = k;
            iout[pos] = si[lp];
        }
    }
}

// p_r = exp((double) w_r - w_0) over the sorted ranks r < keep (w recomputed
// from the logits as the reference forms it), and per block of SMP_PB ranks
// the sum in a fixed order (4 consecutive ranks per thread, then a tree).
// (Indices are range-checked before use, so a sort fault cannot turn into
// an out-of-bounds read.)
extern "C" __global__ void __launch_bounds__(256)
smp_probs(const float *__restrict__ x, float temp, const int *__restrict__ idx, int n, int keep,
          double *__restrict__ p, double *__restrict__ bsum) {
    __shared__ double red[256];
    const int tid = threadIdx.x, r0 = blockIdx.x * SMP_PB + 4 * tid;
    const int i0 = idx[0];
    const double mx = (double)(x[(unsigned)i0 < (unsigned)n ? i0 : 0] / temp);
    double s = 0.0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int r = r0 + j;
        if (r < keep) {
            const int i = idx[r];
            const double v = exp((double)(x[(unsigned)i < (unsigned)n ? i : 0] / temp) - mx);
            p[r] = v;
            s += v;
        }
    }
    red[tid] = s;
    __syncthreads();
    for (int o = 128; o > 0; o >>= 1) {
        if (tid < o) red[tid] += red[tid + o];
        __syncthreads();
    }
    if (tid == 0) bsum[blockIdx.x] = red[0];
}

struct SmpFinishArgs {
    const float *x;
    float temp;
    int keep;
    float top_p;
    const int *idx;          // sorted indices
    const double *p;         // [keep]
    const double *bsum;      // [nbp]
    int nbp;
    const int *bad;          // [nblk] non-finite flags of the first histogram pass
    int nblk;
    unsigned long long *rng; // xorshift64* state, advanced once
    int *out;                // the id (when pos is null)
    int *ids;                // position-driven: ids[*pos + 1] = id, flag[*pos + 1] = flag, then ++*pos
    int *pos;
    int *flag;               // 0 certified, 1 within the bound of a boundary, 2 non-finite input
    int n;                   // row length (bounds the sorted indices)
};

struct SmpState {
    double bp[SMP_MAXB * SMP_SB / SMP_PB + 1];   // exclusive prefix of the block sums
    double sc[SMP_PB];                            // inclusive scan of one block's q
    double qv[SMP_PB];                            // that block's q
    double wtot[16];
    int first[16];
    double den;
    int nbp, keep, cur;                           // cur: the block held in sc / qv (-1 none)
};

// Lowest thread index whose pred holds (1024 if none).
__device__ __forceinline__ int smp_first(bool pred, SmpState &S) {
    const unsigned long long m = __ballot(pred);
    const int tid = threadIdx.x, w = tid >> 6;
    if ((tid & 63) == 0) S.first[w] = m ? w * 64 + __ffsll((long long)m) - 1 : 1024;
    __syncthreads();
    int r = 1024;
#pragma unroll
    for (int i = 0; i < 16; ++i) r = min(r, S.first[i]);
    __syncthreads();
    return r;
}

// Inclusive scan over the workgroup of one value per thread into S.sc
// (wave shuffles, then the wave totals).
__device__ __forceinline__ void smp_scan_wg(double v, SmpState &S) {
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    double incl = v;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const double t = __shfl_up(incl, o, 64);
        if (lane >= o) incl += t;
    }
    if (lane == 63) S.wtot[w] = incl;
    __syncthreads();
    double pre = 0.0;
    for (int i = 0; i < w; ++i) pre += S.wtot[i];
    S.sc[tid] = pre + incl;
    __syncthreads();
}

// Inclusive scan of q_r = p_r / den over probability block b into S.sc
// (kept while the same block is asked for again); returns this thread's q.
__device__ __forceinline__ double smp_scan_block(int b, const double *__restrict__ p, SmpState &S) {
    const int tid = threadIdx.x;
    if (S.cur == b) return S.qv[tid];
    const int r = b * SMP_PB + tid;
    const double q = r < S.keep ? p[r] / S.den : 0.0;
    S.qv[tid] = q;
    smp_scan_wg(q, S);
    if (tid == 0) S.cur = b;
    __syncthreads();
    return q;
}

// First rank r < keep with F_r = cum_r - q_r > t (cum_r: mass of ranks < r),
// else keep.  Blocks whose last F is at most t - 2 eta cannot hold such a
// rank (F is non-decreasing in exact arithmetic), which skips them.  With
// skip1 (the two largest w equal, t >= 0) rank 1 is never a crossing: its p
// is exp(0) = 1 = p_0 on both sides and cum_1 = q_0 exactly, so F_1 = 0 <= t
// exactly in the reference as here.
__device__ int smp_cross(double t, double eta, bool skip1, const double *__restrict__ p, SmpState &S) {
    const int tid = threadIdx.x;
    bool may = false;
    if (tid < S.nbp) {
        const int re = min(S.keep, (tid + 1) * SMP_PB) - 1;
        const double qe = p[re] / S.den;
        may = (S.bp[tid + 1] - p[re]) / S.den - qe > t - 2.0 * eta;
    }
    for (int b = smp_first(may, S); b < S.nbp; ++b) {
        const double q = smp_scan_block(b, p, S);
        const int r = b * SMP_PB + tid;
        const double cum = S.bp[b] / S.den + (tid ? S.sc[tid - 1] : 0.0);
        const int f = smp_first(r < S.keep && !(skip1 && r == 1) && cum - q > t, S);
        if (f < SMP_PB) return b * SMP_PB + f;
    }
    return S.keep;
}

// Mass of the ranks below n (n <= keep).
__device__ double smp_prefix(int n, const double *__restrict__ p, SmpState &S) {
    if (n >= S.keep) return S.bp[S.nbp] / S.den;
    const int b = n / SMP_PB, t = n % SMP_PB;
    smp_scan_block(b, p, S);
    return S.bp[b] / S.den + (t ? S.sc[t - 1] : 0.0);
}

extern "C" __global__ void __launch_bounds__(1024)
smp_finish(SmpFinishArgs a) {
#pragma clang fp contract(off)
    __shared__ SmpState S;
    __shared__ double Ush;
    const int tid = threadIdx.x;
    if (tid == 0) {
        S.nbp = a.nbp;
        S.keep = a.keep;
        S.cur = -1;
    }
    // exclusive prefix of the block sums (<= 256 blocks)
    smp_scan_wg(tid < a.nbp ? a.bsum[tid] : 0.0, S);
    if (tid <= a.nbp) S.bp[tid] = tid ? S.sc[tid - 1] : 0.0;
    int nf = 0;
    for (int i = tid; i < a.nblk; i += 1024) nf |= a.bad[i];
    const bool nonfinite = smp_first(nf != 0, S) < 1024;   // (also the barrier after the bp writes)
    if (tid == 0) S.den = S.bp[a.nbp];
    __syncthreads();

    const double eps = 1.0 / 9007199254740992.0;   // 2^-53
    const double eta = 8.0 * 4.0 * (2.0 * eps) + 4.0 * ((double)a.keep + 64.0) * eps;
    const double tp = (double)a.top_p;
    const int i0 = a.idx[0], i1 = a.keep >= 2 ? a.idx[1] : i0;
    const bool skip1 = a.keep >= 2 && tp >= 0.0 && (unsigned)i0 < (unsigned)a.n && (unsigned)i1 < (unsigned)a.n &&
                       a.x[i0] / a.temp == a.x[i1] / a.temp;
    // nucleus cut: the reference's nkeep lies in [lo, hi]; nk is the best estimate
    const int nk = smp_cross(tp, eta, skip1, a.p, S);
    const int lo = smp_cross(tp - 2.0 * eta, eta, skip1, a.p, S);
    const int hi = smp_cross(tp + 2.0 * eta, eta, skip1, a.p, S);
    const double mass = smp_prefix(nk, a.p, S);
    const double mass_lo = smp_prefix(lo, a.p, S), mass_hi = smp_prefix(hi, a.p, S);
    if (tid == 0) {
        unsigned long long s = *a.rng;
        s ^= s >> 12;
        s ^= s << 25;
        s ^= s >> 27;
        *a.rng = s;
        Ush = (double)((s * 0x2545F4914F6CDD1DULL) >> 11) * eps;
    }
    __syncthreads();
    const double U = Ush, u = U * mass;
    // the draw: first rank r < nk with u <= acc_r (mass of ranks <= r), else nk - 1
    int pick = nk > 0 ? nk - 1 : 0;
    double acc_prev = 0.0, acc_pick = 0.0;
    bool found = false;
    {
        bool may = false;
        if (tid < S.nbp) may = tid * SMP_PB < nk && S.bp[tid + 1] / S.den >= u - 2.0 * eta;
        for (int b = smp_first(may, S); b < S.nbp && b * SMP_PB < nk; ++b) {
            const double q = smp_scan_block(b, a.p, S);
            const int r = b * SMP_PB + tid;
            const double cum = S.bp[b] / S.den + (tid ? S.sc[tid - 1] : 0.0);
            const int f = smp_first(r < nk && u <= cum + q, S);
            if (f < SMP_PB) {
                pick = b * SMP_PB + f;
                acc_prev = S.bp[b] / S.den + (f ? S.sc[f - 1] : 0.0);
                acc_pick = acc_prev + a.p[pick] / S.den;
                found = true;
                break;
            }
        }
    }
    if (!found && nk > 0) acc_prev = smp_prefix(nk - 1, a.p, S) + a.p[nk - 1] / S.den;   // acc of nk - 1
    __syncthreads();
    if (tid == 0) {
        // u_ref lies in [u_lo, u_hi] for every nkeep in [lo, hi]; acc_ref within 2 eta of ours
        const double u_lo = U * fmin(mass_lo, mass_hi) - 2.0 * eta - eps;
        const double u_hi = U * fmax(mass_lo, mass_hi) + 2.0 * eta + eps;
        bool ok;
        if (found)
            ok = pick < lo && (pick == 0 || u_lo - 2.0 * eta > acc_prev) && u_hi + 2.0 * eta <= acc_pick;
        else
            ok = lo == hi && nk > 0 && u_lo - 2.0 * eta > acc_prev;
        const int id = nk > 0 ? a.idx[pick] : 0;
        const int fl = nonfinite ? 2 : (ok ? 0 : 1);
        if (a.pos) {
            const int ps = *a.pos;
            a.ids[ps + 1] = id;
            a.flag[ps + 1] = fl;
            *a.pos = ps + 1;
        } else {
            *a.out = id;
            *a.flag = fl;
        }
    }
}
