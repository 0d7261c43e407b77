// gfx950 sampler: the reference's qm_sample (src/sampler.c:50-106), token for token and rng state
// for rng state.
//
// The reference's result hangs on two serial double accumulations of floats: the normaliser
// sum += p[i] in index order (src/sampler.c:57-61), whose last bits decide every rounding of
// (float)(p[i] / sum), and the cumulative mass over the sorted candidates (src/sampler.c:89-104),
// which decides the nucleus and the drawn index. Both are computed here exactly, in parallel:
//
//   * the sequence is cut into chunks of 64*J consecutive elements (at most 1024 chunks), each
//     handled by one wave with coalesced loads; a scan of the chunk sums gives every chunk an
//     approximate start a0 and end a1 (relative error below 2^-27 for n <= 2^24);
//   * while the serial sum s stays inside one binade [2^e, 2^(e+1)), adding v rounds v alone to a
//     multiple of ulp = 2^(e-52): s' = s + RNE(v), order-free, except at an exact tie, where
//     round-half-even looks at the parity of s/ulp. A chunk whose a0 and a1 lie in the same binade
//     with a margin (twice that bound) keeps the serial sum in it, and its effect on s is a function of
//     the incoming parity only: (increment, outgoing parity) for parity 0 and for parity 1. Without
//     ties that is one exact sum of the rounded increments; with ties an ordered scan over lanes;
//   * those functions compose associatively, so one segmented scan over chunks gives each chunk the
//     composition since the last chunk that could not be certified (a binade change, a margin miss,
//     or the first nonzero chunk); one wave replays the uncertified chunks serially, in order, from
//     their exact entry value (typically ~10 of the chunks) with the reference's own `s += v`;
//   * every chunk's exact start and end follow; a search for the first prefix reaching a threshold
//     finds its chunk from the ends and replays that one chunk.
//
// Candidates are sorted by (probability descending, index ascending) with a stable LSD radix sort
// on the probability bits (the heap of src/sampler.c:75-87 produces exactly this order: its less()
// is a total order when no probability is NaN). A NaN probability makes the reference's sum NaN,
// every probability NaN, and its heap then returns index 0 after drawing once: handled directly.
//
// Small vocabularies run as one 1024-thread workgroup (k_sample). Larger ones run as a chain of
// kernels, one per global dependency (a kernel boundary is cheaper here than a device-scope fence):
//   exp + chunk sums | chunk transfers | walk -> normaliser (one workgroup) | probabilities +
//   candidate counts | stable compaction + first digit histogram | 4 radix passes (each builds the
//   next histogram) | nucleus chunk sums | nucleus transfers | walk, searches, rng, token (one
//   workgroup).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <mutex>

#include "qmh_device.h"
#include "qmh_launch.h"

namespace {

constexpr int MAXCH = 1024;  // chunks of an exact sum
constexpr int NONE = 0x7fffffff;
constexpr int CL_REPLAY = -10000, CL_ZERO = -20000;  // chunk classes besides a binade exponent
constexpr int SMALL_N = 8192;                         // single-workgroup path up to this vocabulary
constexpr int GT = 256;                               // grid path: threads per workgroup
constexpr int TILE = 1024;                            // grid radix sort: elements per workgroup
constexpr int STAGE_F = 4096;                         // staged values of replayed chunks

// ---------------------------------------------------------------- block helpers (NT threads)

template <int NT>
__device__ __forceinline__ int block_exscan_i(int v, int *wbuf, int *total) {
    constexpr int NW = NT / 64;
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    int x = v;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const int y = __shfl_up(x, o);
        if (lane >= o) x += y;
    }
    if (lane == 63) wbuf[w] = x;
    __syncthreads();
    int pre = 0, tot = 0;
#pragma unroll
    for (int k = 0; k < NW; k++) {
        const int t = wbuf[k];
        pre += k < w ? t : 0;
        tot += t;
    }
    __syncthreads();
    *total = tot;
    return pre + x - v;
}

// approximate (any fixed order): only used to place chunks in binades, with a certified margin
template <int NT>
__device__ __forceinline__ double block_exscan_d(double v, double *wbuf) {
    constexpr int NW = NT / 64;
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    double x = v;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const double y = __shfl_up(x, o);
        if (lane >= o) x += y;
    }
    if (lane == 63) wbuf[w] = x;
    double ex = __shfl_up(x, 1);  // exclusive by a lane shift (x - v would lose small prefixes)
    if (lane == 0) ex = 0.0;
    __syncthreads();
    double pre = 0.0;
#pragma unroll
    for (int k = 0; k < NW; k++)
        if (k < w) pre += wbuf[k];
    __syncthreads();
    return pre + ex;
}

template <int NT>
__device__ __forceinline__ int block_min_i(int v, int *wbuf) {
    constexpr int NW = NT / 64;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = min(v, __shfl_xor(v, o));
    if ((threadIdx.x & 63) == 0) wbuf[threadIdx.x >> 6] = v;
    __syncthreads();
    int r = wbuf[0];
#pragma unroll
    for (int k = 1; k < NW; k++) r = min(r, wbuf[k]);
    __syncthreads();
    return r;
}

template <int NT>
__device__ __forceinline__ float block_max_f(float v, float *wbuf) {
    constexpr int NW = NT / 64;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float y = __shfl_xor(v, o);
        v = y > v ? y : v;
    }
    if ((threadIdx.x & 63) == 0) wbuf[threadIdx.x >> 6] = v;
    __syncthreads();
    float r = wbuf[0];
#pragma unroll
    for (int k = 1; k < NW; k++) r = wbuf[k] > r ? wbuf[k] : r;
    __syncthreads();
    return r;
}

template <int NT>
__device__ __forceinline__ int block_or_i(int v, int *wbuf) {
    constexpr int NW = NT / 64;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v |= __shfl_xor(v, o);
    if ((threadIdx.x & 63) == 0) wbuf[threadIdx.x >> 6] = v;
    __syncthreads();
    int r = 0;
#pragma unroll
    for (int k = 0; k < NW; k++) r |= wbuf[k];
    __syncthreads();
    return r;
}

// exclusive prefix of arr[0..len) into out[] (approximate, fixed order); block-wide call
template <int NT>
__device__ void lds_exscan_d(const double *arr, double *out, int len, double *wbuf) {
    const int t = threadIdx.x, per = (len + NT - 1) / NT, lo = min(t * per, len), hi = min(lo + per, len);
    double s = 0.0;
    for (int i = lo; i < hi; i++) s += arr[i];
    double run = block_exscan_d<NT>(s, wbuf);
    for (int i = lo; i < hi; i++) {
        out[i] = run;
        run += arr[i];
    }
    __syncthreads();
}

// exclusive prefix of arr[0..len) in place (exact); *total gets the sum; block-wide call
template <int NT>
__device__ void lds_exscan_i(int *arr, int len, int *wbuf, int *total) {
    const int t = threadIdx.x, per = (len + NT - 1) / NT, lo = min(t * per, len), hi = min(lo + per, len);
    int s = 0;
    for (int i = lo; i < hi; i++) s += arr[i];
    int run = block_exscan_i<NT>(s, wbuf, total);
    for (int i = lo; i < hi; i++) {
        const int v = arr[i];
        arr[i] = run;
        run += v;
    }
    __syncthreads();
}

// lanes below this one that are set in mask
__device__ __forceinline__ int lanes_below(uint64_t mask) {
    return __builtin_amdgcn_mbcnt_hi((uint32_t)(mask >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)mask, 0));
}

// the lanes holding the same 8-bit digit as this one (among the valid lanes), from 8 ballots
__device__ __forceinline__ uint64_t digit_peers(uint32_t d, bool valid) {
    uint64_t peers = __ballot(valid);
#pragma unroll
    for (int bit = 0; bit < 8; bit++) {
        const uint64_t bb = __ballot((d >> bit) & 1u);
        peers &= ((d >> bit) & 1u) ? bb : ~bb;
    }
    return peers;
}

// ---------------------------------------------------------------- exact serial double sums

// binade exponent of a positive normal double
__device__ __forceinline__ int binade(double a) { return (int)((__double_as_longlong(a) >> 52) & 0x7ff) - 1023; }

// The approximate chunk start / end a differs from the serial value s by at most (len + J + 40) u a
// (u = 2^-53): the serial recursive sum is within (len-1) u of the exact sum, a within (J + 40) u
// (J-term lane sums, a 6-level wave tree, a scan of at most 4 + 6 + 16 levels, one add), every term
// nonnegative. Twice that bound is the margin that certifies s's binade from a.
__device__ __forceinline__ double band_margin(int len) { return (double)(2 * len + 4096) * 0x1p-53; }
__device__ __forceinline__ bool band_certified(double a, int e, double mu) {
    return a >= ldexp(1.0, e) * (1.0 + mu) && a <= ldexp(1.0, e + 1) * (1.0 - mu);
}

// chunk class from its approximate start and end
__device__ __forceinline__ int chunk_class(double a0, double a1, double mu) {
    if (a1 == 0.0) return CL_ZERO;
    if (a0 == 0.0) return CL_REPLAY;
    const int e = binade(a0);
    return (binade(a1) == e && band_certified(a0, e, mu) && band_certified(a1, e, mu)) ? e : CL_REPLAY;
}

// a transfer (i0, i1) applied to an exact serial value s (s = 0 only before the first nonzero
// chunk, where every certified chunk is all zeros)
__device__ __forceinline__ double xfer_apply(long long i0, long long i1, double s) {
    if (s == 0.0) return 0.0;
    const long long inc = (__double_as_longlong(s) & 1) ? i1 : i0;
    return s + (double)inc * ldexp(1.0, binade(s) - 52);
}

// (a then b); bit2 of the out bits marks a reset (a replayed chunk): composition restarts after it
__device__ __forceinline__ void xfer_then(long long &a0, long long &a1, int &ao, long long b0, long long b1, int bo) {
    if (bo & 4) {
        a0 = b0;
        a1 = b1;
        ao = bo;
        return;
    }
    const int q0 = ao & 1, q1 = (ao >> 1) & 1;
    a0 += q0 ? b1 : b0;
    a1 += q1 ? b1 : b0;
    ao = (ao & 4) | ((bo >> q0) & 1) | (((bo >> q1) & 1) << 1);
}

// approximate sum of chunk c (elements c*ch + k*64 + lane), all lanes get it
template <class Get>
__device__ __forceinline__ double wave_chunk_sum(const Get &get, int c, int J, int len) {
    const int lane = threadIdx.x & 63;
    double s = 0.0;
    for (int k = 0; k < J; k++) {
        const int i = c * 64 * J + k * 64 + lane;
        s += i < len ? (double)get(i) : 0.0;
    }
    return qmh_wave_sum_d(s);
}

// transfer of chunk c of class cl (one wave; all lanes get it)
template <class Get>
__device__ void wave_chunk_transfer(const Get &get, int c, int J, int len, int cl, long long &g0, long long &g1,
                                    int &go) {
    const int lane = threadIdx.x & 63;
    g0 = 0;
    g1 = 0;
    go = 2;  // identity
    if (cl == CL_REPLAY) {
        go = 4 | 2;
        return;
    }
    if (cl == CL_ZERO) return;
    const double scale = ldexp(1.0, 52 - cl);  // v / ulp, exact
    double rs = 0.0;
    bool ties = false;
    for (int k = 0; k < J; k++) {
        const int i = c * 64 * J + k * 64 + lane;
        const double y = i < len ? (double)get(i) * scale : 0.0;
        const double fl = floor(y), fr = y - fl;
        ties |= __ballot(fr == 0.5) != 0;
        rs += fl + (fr > 0.5 ? 1.0 : 0.0);
    }
    if (!ties) {  // one exact sum: all partial sums are integers below 2^52
        const long long r = (long long)qmh_wave_sum_d(rs);
        g0 = r;
        g1 = r;
        go = (int)(r & 1) | ((int)((r + 1) & 1) << 1);
        return;
    }
    for (int k = 0; k < J; k++) {  // round-half-even at ties: ordered composition over lanes, then k
        const int i = c * 64 * J + k * 64 + lane;
        const double y = i < len ? (double)get(i) * scale : 0.0;
        const double fl = floor(y), fr = y - fl;
        const long long a = (long long)fl;
        long long e0, e1;
        int eo;
        if (fr == 0.5) {  // x -> x + a rounded up to even
            e0 = a + (a & 1);
            e1 = a + ((a + 1) & 1);
            eo = 0;
        } else {
            const long long r = a + (fr > 0.5 ? 1 : 0);
            e0 = r;
            e1 = r;
            eo = (int)(r & 1) | ((int)((r + 1) & 1) << 1);
        }
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {  // inclusive scan over lanes
            const long long y0 = __shfl_up(e0, o), y1 = __shfl_up(e1, o);
            const int yo = __shfl_up(eo, o);
            if (lane >= o) {
                long long n0 = y0, n1 = y1;
                int no = yo;
                xfer_then(n0, n1, no, e0, e1, eo);
                e0 = n0;
                e1 = n1;
                eo = no;
            }
        }
        const long long t0 = __shfl(e0, 63), t1 = __shfl(e1, 63);
        const int to = __shfl(eo, 63);
        xfer_then(g0, g1, go, t0, t1, to);
    }
}

// serial replay by one wave of elements [lo, hi) from the exact value s: every lane ends with the
// same s; *hit gets the first index whose running value passes test, or NONE
template <class Get, class Test>
__device__ double wave_replay(const Get &get, int lo, int hi, double s, const Test &test, int *hit) {
    const int lane = threadIdx.x & 63;
    int h = NONE;
    for (int b = lo; b < hi; b += 64) {
        const float v = b + lane < hi ? get(b + lane) : 0.0f;  // lanes past the end add +0: no change
        const int nb = min(64, hi - b);
        for (int q0 = 0; q0 < nb; q0 += 8) {
            double vv[8];
#pragma unroll
            for (int k = 0; k < 8; k++)  // fetched ahead: only the adds are serial
                vv[k] = (double)__int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), q0 + k));
#pragma unroll
            for (int k = 0; k < 8; k++) {
                s += vv[k];
                if (h == NONE && q0 + k < nb && test(s)) h = b + q0 + k;
            }
        }
    }
    *hit = h;
    return s;
}

// chunk-level state of one exact sum (LDS)
struct ExSums {
    double csum[MAXCH];              // approximate chunk sums
    int cls[MAXCH];                  // binade exponent, CL_REPLAY or CL_ZERO
    long long f0[MAXCH], f1[MAXCH];  // chunk transfer: increment for incoming parity 0 / 1
    int fo[MAXCH];                   // bit0/bit1: outgoing parity for 0/1, bit2: replayed chunk
    long long p0[MAXCH], p1[MAXCH];  // segmented exclusive prefix of the transfers
    int xo[MAXCH];                   // replayed chunks before this one
    int xlist[MAXCH];                // replayed chunks in order
    double xin[MAXCH], xout[MAXCH];  // their exact entry / exit values
    double start[MAXCH], end[MAXCH];  // every chunk's exact start / end (start: also the approximate
                                      // prefix while classifying)
    float stage[STAGE_F];             // values of the first replayed chunks, fetched in parallel
    double wd[16];
    int wi[16];
    long long pw0[16], pw1[16];  // wave totals of the transfer scan
    int pwo[16];
    double total;
    int nch, nx, status, ires;
};

// exclusive segmented scan of per-thread transfer aggregates over the workgroup (thread order);
// w0/w1/wo: LDS for NT/64 wave totals. Block-wide call.
template <int NT>
__device__ void block_xfer_exscan(long long &c0, long long &c1, int &co, long long *w0, long long *w1, int *wo) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {  // inclusive over the wave
        const long long y0 = __shfl_up(c0, o), y1 = __shfl_up(c1, o);
        const int yo = __shfl_up(co, o);
        if (lane >= o) {
            long long n0 = y0, n1 = y1;
            int no = yo;
            xfer_then(n0, n1, no, c0, c1, co);
            c0 = n0;
            c1 = n1;
            co = no;
        }
    }
    if (lane == 63) {
        w0[w] = c0;
        w1[w] = c1;
        wo[w] = co;
    }
    long long e0 = __shfl_up(c0, 1), e1 = __shfl_up(c1, 1);  // exclusive within the wave
    int eo = __shfl_up(co, 1);
    if (lane == 0) {
        e0 = 0;
        e1 = 0;
        eo = 2;
    }
    __syncthreads();
    if (w == 0) {  // exclusive scan of the wave totals by the first wave
        constexpr int NW = NT / 64;
        long long t0 = lane < NW ? w0[lane] : 0, t1 = lane < NW ? w1[lane] : 0;
        int to = lane < NW ? wo[lane] : 2;
#pragma unroll
        for (int o = 1; o < NW; o <<= 1) {
            const long long y0 = __shfl_up(t0, o), y1 = __shfl_up(t1, o);
            const int yo = __shfl_up(to, o);
            if (lane >= o) {
                long long n0 = y0, n1 = y1;
                int no = yo;
                xfer_then(n0, n1, no, t0, t1, to);
                t0 = n0;
                t1 = n1;
                to = no;
            }
        }
        long long x0 = __shfl_up(t0, 1), x1 = __shfl_up(t1, 1);
        int xo = __shfl_up(to, 1);
        if (lane < NW) {
            w0[lane] = lane == 0 ? 0 : x0;
            w1[lane] = lane == 0 ? 0 : x1;
            wo[lane] = lane == 0 ? 2 : xo;
        }
    }
    __syncthreads();
    long long q0 = w0[w], q1 = w1[w];
    int qo = wo[w];
    xfer_then(q0, q1, qo, e0, e1, eo);
    __syncthreads();
    c0 = q0;
    c1 = q1;
    co = qo;
}

// From the chunk classes and transfers in x: the segmented scan, the serial walk over replayed
// chunks, every chunk's exact start / end and the total. A certified chunk whose transfer leaves its
// binade, or a chunk end that is not the next chunk's start, sets `bad` in x.status (never
// expected); the starts, ends and total are then recomputed by one serial pass in the reference's
// order, so the result stays exact. force: take that serial pass unconditionally (a host switch
// that lets tests run it). Block-wide call.
template <int NT, class Get>
__device__ void finish_sums(const Get &get, int len, int ch, int nch, ExSums &x, int bad, bool force) {
    const int t = threadIdx.x, lane = t & 63;
    {
        // thread t composes chunks [t*per, t*per+per), then one scan over the threads
        const int per = (nch + NT - 1) / NT, lo = min(t * per, nch), hi = min(lo + per, nch);
        long long c0 = 0, c1 = 0;
        int co = 2, cx = 0;
        for (int i = lo; i < hi; i++) {
            xfer_then(c0, c1, co, x.f0[i], x.f1[i], x.fo[i]);
            cx += x.cls[i] == CL_REPLAY;
        }
        block_xfer_exscan<NT>(c0, c1, co, x.pw0, x.pw1, x.pwo);
        int nx;
        int qx = block_exscan_i<NT>(cx, x.wi, &nx);
        for (int i = lo; i < hi; i++) {
            x.p0[i] = c0;
            x.p1[i] = c1;
            x.xo[i] = qx;
            if (x.cls[i] == CL_REPLAY) x.xlist[qx++] = i;
            xfer_then(c0, c1, co, x.f0[i], x.f1[i], x.fo[i]);
        }
        if (t == 0) x.nx = nx;
    }
    __syncthreads();
    // the replayed chunks' values, as many as fit, fetched by the whole workgroup at once
    const int nx = x.nx, nst = min(nx, STAGE_F / ch);
    for (int j = t; j < nst * ch; j += NT) {
        const int i = x.xlist[j / ch] * ch + j % ch;
        x.stage[j] = i < len ? get(i) : 0.0f;
    }
    __syncthreads();
    if (t < 64) {
        // serial walk over the replayed chunks, one wave: the sum runs in order
        double s = 0.0;
        for (int k = 0; k < nx; k++) {
            const int c = __builtin_amdgcn_readfirstlane(x.xlist[k]);
            const double sin = xfer_apply(x.p0[c], x.p1[c], s);
            const int clo = c * ch, chi = min(clo + ch, len);
            int dummy;
            if (k < nst) {
                const float *sv = x.stage + k * ch;
                s = wave_replay([&](int i) { return sv[i - clo]; }, clo, chi, sin, [](double) { return false; },
                                &dummy);
            } else {
                s = wave_replay(get, clo, chi, sin, [](double) { return false; }, &dummy);
            }
            if (lane == 0) {
                x.xin[k] = sin;
                x.xout[k] = s;
            }
        }
    }
    __syncthreads();
    for (int c = t; c < nch; c += NT) {
        const int cl = x.cls[c], xo = x.xo[c];
        double st, en;
        if (cl == CL_REPLAY) {
            st = x.xin[xo];
            en = x.xout[xo];
        } else {
            st = xfer_apply(x.p0[c], x.p1[c], xo > 0 ? x.xout[xo - 1] : 0.0);
            en = xfer_apply(x.f0[c], x.f1[c], st);
            const bool ok = cl == CL_ZERO ? (st == 0.0 && en == 0.0) : (binade(st) == cl && binade(en) == cl);
            if (!ok) atomicOr(&x.status, bad);
        }
        x.start[c] = st;
        x.end[c] = en;
    }
    __syncthreads();
    for (int c = t; c + 1 < nch; c += NT)
        if (x.end[c] != x.start[c + 1]) atomicOr(&x.status, bad);
    if (t == 0) {
        if (force) x.status |= bad;
        x.total = nch > 0 ? x.end[nch - 1] : 0.0;
        x.nch = nch;
    }
    __syncthreads();
    if (x.status & bad) {  // uniform: the serial sum s += v over every element, chunk by chunk
        if (t < 64) {
            double s = 0.0;
            for (int c = 0; c < nch; c++) {
                if (lane == 0) x.start[c] = s;
                int dummy;
                s = wave_replay(get, c * ch, min(c * ch + ch, len), s, [](double) { return false; }, &dummy);
                if (lane == 0) x.end[c] = s;
            }
            if (lane == 0) x.total = nch > 0 ? s : 0.0;
        }
        __syncthreads();
    }
}

// chunk geometry of an exact sum over len elements
__device__ __forceinline__ int chunk_j(int len) { return max(1, (len + 64 * MAXCH - 1) / (64 * MAXCH)); }

// first index i of [0, lim) (lim <= len) whose exact inclusive prefix passes test (monotone in
// the prefix), or NONE: the chunk from the ends, then one wave replays it. Block-wide call.
template <int NT, class Get, class Test>
__device__ int exact_first(const Get &get, int ch, int lim, ExSums &x, const Test &test) {
    const int t = threadIdx.x;
    int best = NONE;
    for (int c = t; c < x.nch; c += NT)
        if (c * ch < lim && test(x.end[c])) {
            best = c;
            break;
        }
    const int c = block_min_i<NT>(best, x.wi);
    if (c != NONE && t < 64) {
        int h;
        wave_replay(get, c * ch, min(c * ch + ch, lim), x.start[c], test, &h);
        if (t == 0) x.ires = h;
    }
    __syncthreads();
    const int r = c == NONE ? NONE : x.ires;
    __syncthreads();
    return r;
}

// the exact prefix through index m-1 (m >= 1): one wave replays the chunk of m-1. Block-wide call.
template <class Get>
__device__ double exact_prefix(const Get &get, int ch, int m, ExSums &x) {
    if (threadIdx.x < 64) {
        const int c = (m - 1) / ch;
        int dummy;
        const double s = wave_replay(get, c * ch, m, x.start[c], [](double) { return false; }, &dummy);
        if (threadIdx.x == 0) x.total = s;
    }
    __syncthreads();
    const double r = x.total;
    __syncthreads();
    return r;
}

// ---------------------------------------------------------------- shared by both paths

__device__ __forceinline__ float rng_uniform(uint64_t *state) {  // xorshift64* (src/sampler.c:18-25)
    uint64_t x = *state;
    x ^= x >> 12;
    x ^= x << 25;
    x ^= x >> 27;
    *state = x;
    return (float)((x * 0x2545F4914F6CDD1DULL) >> 40) / 16777216.0f;
}

__device__ __forceinline__ void emit(const qmh_sample_args &a, int tok) {
    if (a.out) *a.out = tok;
    if (a.tokpos) {
        a.tokpos[0] = tok;
        a.tokpos[1] += 1;
        const int step = a.tokpos[2];
        if (a.record && step >= 0 && step < a.record_cap) a.record[step] = tok;
        a.tokpos[2] = step + 1;
    }
}

// the candidate test of src/sampler.c:66-71: prefilter cut (when it applies) on the probability
__device__ __forceinline__ bool prefilter_on(const qmh_sample_args &a) {
    return a.top_k == 0 && a.top_p < 1.0f && a.n > 1;
}
__device__ __forceinline__ float prefilter_cut(const qmh_sample_args &a) {
    return (1.0f - a.top_p) / (float)(a.n - 1);
}

// probability from a sort key (key = bits(1.0f) - bits(q): ascending key = descending q)
__device__ __forceinline__ uint32_t prob_key(float q) { return 0x3f800000u - __float_as_uint(q); }
__device__ __forceinline__ float key_prob(uint32_t k) { return __uint_as_float(0x3f800000u - k); }

// ---------------------------------------------------------------- single-workgroup path

constexpr int NT1 = 1024, NW1 = NT1 / 64;

struct SmallShared {
    ExSums x;
    uint32_t cnt[256 * NW1];  // radix-sort counters per (digit, wave), digit-major
    float wf[NW1];
    int wi[NW1];
    double res;
};

__global__ __launch_bounds__(NT1) void k_sample(qmh_sample_args a) {
    __shared__ SmallShared sh;
    ExSums &x = sh.x;
    const int t = threadIdx.x, lane = t & 63, w = t >> 6, n = a.n;
    if (t == 0) x.status = 0;
    // ---- exponentials (src/sampler.c:54-61): max by strict-greater scan from logits[0]
    float v = -__builtin_inff();
    for (int i0 = 1 + t; i0 < n; i0 += 8 * NT1) {  // 8 loads in flight
        float l[8];
#pragma unroll
        for (int k = 0; k < 8; k++) l[k] = i0 + k * NT1 < n ? a.logits[i0 + k * NT1] : -__builtin_inff();
#pragma unroll
        for (int k = 0; k < 8; k++) v = l[k] > v ? l[k] : v;  // NaNs never win
    }
    v = block_max_f<NT1>(v, sh.wf);
    const float l0 = a.logits[0];
    const float mx = v > l0 ? v : l0;  // a NaN logits[0] stays the maximum, as in the serial scan
    const float T = a.temperature;
    int nan = 0;
    for (int i = t; i < n; i += NT1) {
        const float p = qmh_expf((a.logits[i] - mx) / T);
        nan |= p != p;
        a.p[i] = p;
    }
    nan = block_or_i<NT1>(nan, sh.wi);
    float u01 = 0.0f;
    if (t == 0) {
        uint64_t st = *a.rng;
        u01 = rng_uniform(&st);  // one draw per non-greedy call (src/sampler.c:100)
        *a.rng = st;
    }
    if (nan) {  // the reference's sum is NaN and its heap returns index 0
        if (t == 0) {
            emit(a, 0);
            if (a.diag) {
                a.diag[0] = __builtin_nan("");
                a.diag[1] = 0;
            }
        }
        return;
    }
    __syncthreads();  // a.p visible to the workgroup
    // ---- exact serial normaliser (src/sampler.c:57-61)
    const float *pv = a.p;
    auto getp = [&](int i) { return pv[i]; };
    {
        const int J = chunk_j(n), ch = 64 * J, nch = (n + ch - 1) / ch;
        for (int c = w; c < nch; c += NW1) {
            const double s = wave_chunk_sum(getp, c, J, n);
            if (lane == 0) x.csum[c] = s;
        }
        __syncthreads();
        lds_exscan_d<NT1>(x.csum, x.start, nch, x.wd);
        for (int c = t; c < nch; c += NT1) x.cls[c] = chunk_class(x.start[c], x.start[c] + x.csum[c], band_margin(n));
        __syncthreads();
        for (int c = w; c < nch; c += NW1) {
            long long g0, g1;
            int go;
            wave_chunk_transfer(getp, c, J, n, __builtin_amdgcn_readfirstlane(x.cls[c]), g0, g1, go);
            if (lane == 0) {
                x.f0[c] = g0;
                x.f1[c] = g1;
                x.fo[c] = go;
            }
        }
        __syncthreads();
        finish_sums<NT1>(getp, n, ch, nch, x, 1, a.force_serial != 0);
    }
    const double S = x.total;
    const int nx_sum = x.nx;
    // ---- candidates in index order (src/sampler.c:62-75): probabilities, then wave w compacts the
    //      contiguous range [w*R, w*R+R) with ballots, so the order is the index order
    const bool pre = prefilter_on(a);
    const float cut = pre ? prefilter_cut(a) : 0.0f;
    const int R = ((n + NW1 - 1) / NW1 + 63) & ~63;
    const int rlo = min(w * R, n), rhi = min(rlo + R, n);
    int wc = 0;
    for (int b = rlo; b < rhi; b += 64) {
        const int i = b + lane;
        bool c = false;
        if (i < rhi) {
            const float q = (float)((double)a.p[i] / S);  // src/sampler.c:62
            a.p[i] = q;
            c = !pre || q >= cut;
        }
        wc += __popcll(__ballot(c));
    }
    if (lane == 0) sh.wi[w] = wc;
    __syncthreads();
    int nc = 0, off = 0;
#pragma unroll
    for (int k = 0; k < NW1; k++) {
        off += k < w ? sh.wi[k] : 0;
        nc += sh.wi[k];
    }
    __syncthreads();
    const bool all = nc == 0 || !pre;
    if (all) {
        nc = n;
        off = rlo;
    }
    uint32_t kor = 0, kand = 0xffffffffu;
    for (int b = rlo; b < rhi; b += 64) {
        const int i = b + lane;
        const float q = i < rhi ? a.p[i] : 0.0f;
        const bool c = i < rhi && (all || q >= cut);
        const uint64_t m = __ballot(c);
        if (c) {
            const uint32_t key = prob_key(q);
            const int pos = off + lanes_below(m);
            a.key0[pos] = key;
            a.idx0[pos] = i;
            kor |= key;
            kand &= key;
        }
        off += __popcll(m);
    }
    // key bits that differ between candidates: a byte with none is the same for all, no pass
    const uint32_t any1 = (uint32_t)block_or_i<NT1>((int)kor, sh.wi);
    const uint32_t all1 = ~(uint32_t)block_or_i<NT1>((int)~kand, sh.wi);
    const uint32_t diff = any1 ^ all1;
    // ---- stable LSD radix sort of the candidates, 8-bit digits. Wave w ranks the contiguous range
    //      [w*R3, w*R3+R3) 64 elements at a time: the lanes holding digit d find each other from 8
    //      ballots of the digit bits; the lowest of them adds the group's size to the counter.
    uint32_t *ks = a.key0, *kd = a.key1;
    int32_t *is = a.idx0, *id = a.idx1;
    const int R3 = ((nc + NW1 - 1) / NW1 + 63) & ~63;
    const int slo = min(w * R3, nc), shi = min(slo + R3, nc);
    for (int sft = 0; sft < 32; sft += 8) {
        if (((diff >> sft) & 255u) == 0) continue;
        for (int k = t; k < 256 * NW1; k += NT1) sh.cnt[k] = 0;
        __syncthreads();
        for (int b = slo; b < shi; b += 64) {
            const int i = b + lane;
            const bool valid = i < shi;
            const uint32_t d = valid ? (ks[i] >> sft) & 255u : 0u;
            const uint64_t peers = digit_peers(d, valid);
            if (valid && lanes_below(peers) == 0) sh.cnt[d * NW1 + w] += (uint32_t)__popcll(peers);
        }
        __syncthreads();
        uint32_t c4[4], tot = 0;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            c4[k] = sh.cnt[4 * t + k];
            tot += c4[k];
        }
        int dummy;
        uint32_t run = (uint32_t)block_exscan_i<NT1>((int)tot, sh.wi, &dummy);
#pragma unroll
        for (int k = 0; k < 4; k++) {
            sh.cnt[4 * t + k] = run;
            run += c4[k];
        }
        __syncthreads();
        for (int b = slo; b < shi; b += 64) {
            const int i = b + lane;
            const bool valid = i < shi;
            const uint32_t key = valid ? ks[i] : 0u;
            const int32_t ix = valid ? is[i] : 0;
            const uint32_t d = (key >> sft) & 255u;
            const uint64_t peers = digit_peers(d, valid);
            const uint32_t base = valid ? sh.cnt[d * NW1 + w] : 0u;
            const int rank = lanes_below(peers);
            if (valid) {
                kd[base + rank] = key;
                id[base + rank] = ix;
                if (rank == 0) sh.cnt[d * NW1 + w] = base + (uint32_t)__popcll(peers);
            }
        }
        __syncthreads();
        uint32_t *tk = ks;
        ks = kd;
        kd = tk;
        int32_t *ti = is;
        is = id;
        id = ti;
    }
    // ---- nucleus over the k best (src/sampler.c:88-105): exact serial cumulative mass
    const int kk = (a.top_k > 0 && a.top_k < nc) ? a.top_k : nc;
    const uint32_t *kv = ks;
    auto getq = [&](int i) { return key_prob(kv[i]); };
    const int J2 = chunk_j(kk), ch2 = 64 * J2, nch2 = (kk + ch2 - 1) / ch2;
    for (int c = w; c < nch2; c += NW1) {
        const double s = wave_chunk_sum(getq, c, J2, kk);
        if (lane == 0) x.csum[c] = s;
    }
    __syncthreads();
    lds_exscan_d<NT1>(x.csum, x.start, nch2, x.wd);
    for (int c = t; c < nch2; c += NT1) x.cls[c] = chunk_class(x.start[c], x.start[c] + x.csum[c], band_margin(kk));
    __syncthreads();
    for (int c = w; c < nch2; c += NW1) {
        long long g0, g1;
        int go;
        wave_chunk_transfer(getq, c, J2, kk, __builtin_amdgcn_readfirstlane(x.cls[c]), g0, g1, go);
        if (lane == 0) {
            x.f0[c] = g0;
            x.f1[c] = g1;
            x.fo[c] = go;
        }
    }
    __syncthreads();
    finish_sums<NT1>(getq, kk, ch2, nch2, x, 2, a.force_serial != 0);
    const int nx_nuc = x.nx;
    const double tp = (double)a.top_p;
    const int first = exact_first<NT1>(getq, ch2, kk, x, [&](double s) { return s >= tp; });
    const int m = first == NONE ? kk : first + 1;
    const double mass = exact_prefix(getq, ch2, m, x);
    if (t == 0) sh.res = (double)u01 * mass;  // (double)u01 * mass (src/sampler.c:100)
    __syncthreads();
    const double u = sh.res;
    const int hit = exact_first<NT1>(getq, ch2, m, x, [&](double s) { return u < s; });
    if (t == 0) {
        emit(a, is[hit == NONE ? m - 1 : hit]);
        if (a.diag) {
            a.diag[0] = S;
            a.diag[1] = (double)x.status;
            a.diag[2] = (double)nx_sum;
            a.diag[3] = (double)nc;
            a.diag[4] = (double)kk;
            a.diag[5] = (double)m;
            a.diag[6] = (double)nx_nuc;
            a.diag[7] = mass;
        }
    }
}

// ---------------------------------------------------------------- grid path

constexpr int GMAX = MAXCH / (GT / 64);  // workgroups of a chunk kernel
constexpr int NTF = 1024;                // threads of the finishing kernels

// device control block of one draw (at the start of the workspace)
struct Ctl {
    double S;  // exact normaliser
    int nan;   // a NaN exponential: token 0 (cleared by the draw kernel)
    int status, nx_sum;
    int nc, kk, npass;
    int shift[4];
};

struct Ws {
    Ctl *ctl;
    double *csum;
    long long *f0, *f1;
    uint32_t *bits;  // [4][GMAX]: per-workgroup OR / AND of the keys of candidates / of every index
    int *cls, *fo, *ccnt;
    uint32_t *hist;  // [4][ntile_max * 256]
};

__host__ __device__ constexpr size_t ws_align(size_t b) { return (b + 255) & ~(size_t)255; }
__host__ __device__ constexpr int ntile_max(int n) { return (n + TILE - 1) / TILE; }
__host__ __device__ constexpr size_t ws_bytes(int n) {
    return ws_align(sizeof(Ctl)) + ws_align(MAXCH * 8) * 3 + ws_align(4 * GMAX * 4) + ws_align(MAXCH * 4) * 3 +
           ws_align((size_t)4 * ntile_max(n) * 256 * 4);
}
__device__ inline Ws ws_of(const qmh_sample_args &a) {
    uint8_t *p = (uint8_t *)a.ws;
    Ws w;
    w.ctl = (Ctl *)p;
    p += ws_align(sizeof(Ctl));
    w.csum = (double *)p;
    p += ws_align(MAXCH * 8);
    w.f0 = (long long *)p;
    p += ws_align(MAXCH * 8);
    w.f1 = (long long *)p;
    p += ws_align(MAXCH * 8);
    w.bits = (uint32_t *)p;
    p += ws_align(4 * GMAX * 4);
    w.cls = (int *)p;
    p += ws_align(MAXCH * 4);
    w.fo = (int *)p;
    p += ws_align(MAXCH * 4);
    w.ccnt = (int *)p;
    p += ws_align(MAXCH * 4);
    w.hist = (uint32_t *)p;
    return w;
}

__device__ __forceinline__ const uint32_t *sorted_keys(const qmh_sample_args &a, const Ctl *ctl) {
    return (ctl->npass & 1) ? a.key1 : a.key0;
}
__device__ __forceinline__ const int32_t *sorted_idx(const qmh_sample_args &a, const Ctl *ctl) {
    return (ctl->npass & 1) ? a.idx1 : a.idx0;
}

// K1: exponentials and approximate chunk sums of the normaliser; clears the histograms. Each
// workgroup finds the maximum itself (128 KB of L2 reads at vocabulary 32000, cheaper than a
// kernel boundary).
__global__ __launch_bounds__(GT) void k_smp_exp(qmh_sample_args a) {
    __shared__ float wf[GT / 64];
    const Ws ws = ws_of(a);
    const int t = threadIdx.x, lane = t & 63, w = t >> 6, n = a.n;
    const float *lg = a.logits;
    // max over the non-NaN logits, index 0 included; a NaN logits[0] is the serial scan's maximum
    float v = -__builtin_inff();
    if (((uintptr_t)lg & 15) == 0) {
        const int n4 = n >> 2;
        const float4 *l4 = (const float4 *)lg;
        for (int i0 = t; i0 < n4; i0 += 8 * GT) {  // 8 vector loads in flight
            float4 x[8];
#pragma unroll
            for (int k = 0; k < 8; k++)
                x[k] = i0 + k * GT < n4 ? l4[i0 + k * GT]
                                        : make_float4(-__builtin_inff(), -__builtin_inff(), -__builtin_inff(),
                                                      -__builtin_inff());
#pragma unroll
            for (int k = 0; k < 8; k++) {
                v = x[k].x > v ? x[k].x : v;
                v = x[k].y > v ? x[k].y : v;
                v = x[k].z > v ? x[k].z : v;
                v = x[k].w > v ? x[k].w : v;
            }
        }
        for (int i = 4 * n4 + t; i < n; i += GT) v = lg[i] > v ? lg[i] : v;
    } else {
        for (int i0 = t; i0 < n; i0 += 8 * GT) {
            float l[8];
#pragma unroll
            for (int k = 0; k < 8; k++) l[k] = i0 + k * GT < n ? lg[i0 + k * GT] : -__builtin_inff();
#pragma unroll
            for (int k = 0; k < 8; k++) v = l[k] > v ? l[k] : v;
        }
    }
    v = block_max_f<GT>(v, wf);
    const float l0 = lg[0];
    const float mx = l0 != l0 ? l0 : v;
    const int nh = 4 * ntile_max(n) * 256;
    for (int k = blockIdx.x * GT + t; k < nh; k += gridDim.x * GT) ws.hist[k] = 0;
    if (blockIdx.x == 0 && t == 0) ws.ctl->status = 0;
    const int J = chunk_j(n), ch = 64 * J, nch = (n + ch - 1) / ch;
    const int c = blockIdx.x * (GT / 64) + w;
    if (c >= nch) return;
    int nan = 0;
    double s = 0.0;
    for (int k = 0; k < J; k++) {
        const int i = c * ch + k * 64 + lane;
        if (i < n) {
            const float p = qmh_expf((lg[i] - mx) / a.temperature);
            a.p[i] = p;
            nan |= p != p;
            s += (double)p;
        }
    }
    s = qmh_wave_sum_d(s);
    if (lane == 0) ws.csum[c] = s;
    if (__ballot(nan) != 0 && lane == 0) atomicOr(&ws.ctl->nan, 1);
}

// K2 / K7: class and transfer of each chunk of an exact sum (of the exponentials, or of the sorted
// probabilities when NUC); every workgroup scans all chunk sums itself
template <bool NUC>
__global__ __launch_bounds__(GT) void k_smp_xfer(qmh_sample_args a) {
    __shared__ double cs[MAXCH], pre[MAXCH];
    __shared__ double wd[GT / 64];
    const Ws ws = ws_of(a);
    if (ws.ctl->nan) return;
    const int t = threadIdx.x, lane = t & 63, w = t >> 6;
    const int len = NUC ? ws.ctl->kk : a.n;
    const uint32_t *kv = NUC ? sorted_keys(a, ws.ctl) : nullptr;
    const float *pv = a.p;
    auto get = [&](int i) { return NUC ? key_prob(kv[i]) : pv[i]; };
    const int J = chunk_j(len), nch = (len + 64 * J - 1) / (64 * J);
    for (int c = t; c < nch; c += GT) cs[c] = ws.csum[c];
    __syncthreads();
    lds_exscan_d<GT>(cs, pre, nch, wd);
    const int c = blockIdx.x * (GT / 64) + w;
    if (c >= nch) return;
    const int cl = chunk_class(pre[c], pre[c] + cs[c], band_margin(len));
    long long g0, g1;
    int go;
    wave_chunk_transfer(get, c, J, len, cl, g0, g1, go);
    if (lane == 0) {
        ws.cls[c] = cl;
        ws.f0[c] = g0;
        ws.f1[c] = g1;
        ws.fo[c] = go;
    }
}

// the chunk classes and transfers into LDS, then the exact sum (one 1024-thread workgroup)
template <class Get>
__device__ void fin_sums(const Get &get, int len, const Ws &ws, ExSums &x, int bad, bool force) {
    const int t = threadIdx.x;
    const int J = chunk_j(len), ch = 64 * J, nch = (len + ch - 1) / ch;
    if (t == 0) x.status = 0;
    for (int k = t; k < nch; k += NTF) {
        x.cls[k] = ws.cls[k];
        x.f0[k] = ws.f0[k];
        x.f1[k] = ws.f1[k];
        x.fo[k] = ws.fo[k];
    }
    __syncthreads();
    finish_sums<NTF>(get, len, ch, nch, x, bad, force);
}

// K3: the exact normaliser
__global__ __launch_bounds__(NTF) void k_smp_norm(qmh_sample_args a) {
    __shared__ ExSums x;
    const Ws ws = ws_of(a);
    if (ws.ctl->nan) return;
    const float *pv = a.p;
    fin_sums([&](int i) { return pv[i]; }, a.n, ws, x, 1, a.force_serial != 0);
    if (threadIdx.x == 0) {
        ws.ctl->S = x.total;
        ws.ctl->nx_sum = x.nx;
        ws.ctl->status |= x.status;
    }
}

// K4: probabilities, candidate counts per chunk, key bits per workgroup
__global__ __launch_bounds__(GT) void k_smp_prob(qmh_sample_args a) {
    __shared__ int wi[GT / 64];
    const Ws ws = ws_of(a);
    if (ws.ctl->nan) return;
    const int t = threadIdx.x, lane = t & 63, w = t >> 6, n = a.n;
    const double S = ws.ctl->S;
    const bool pre = prefilter_on(a);
    const float cut = pre ? prefilter_cut(a) : 0.0f;
    const int J = chunk_j(n), ch = 64 * J, nch = (n + ch - 1) / ch;
    const int c = blockIdx.x * (GT / 64) + w;
    uint32_t orc = 0, andc = 0xffffffffu, ora = 0, anda = 0xffffffffu;
    if (c < nch) {
        int cnt = 0;
        for (int k = 0; k < J; k++) {
            const int i = c * ch + k * 64 + lane;
            bool cand = false;
            if (i < n) {
                const float q = (float)((double)a.p[i] / S);  // src/sampler.c:62
                a.p[i] = q;
                const uint32_t key = prob_key(q);
                ora |= key;
                anda &= key;
                cand = !pre || q >= cut;
                if (cand) {
                    orc |= key;
                    andc &= key;
                }
            }
            cnt += __popcll(__ballot(cand));
        }
        if (lane == 0) ws.ccnt[c] = cnt;
    }
    orc = (uint32_t)block_or_i<GT>((int)orc, wi);
    ora = (uint32_t)block_or_i<GT>((int)ora, wi);
    andc = ~(uint32_t)block_or_i<GT>((int)~andc, wi);
    anda = ~(uint32_t)block_or_i<GT>((int)~anda, wi);
    if (t == 0) {
        ws.bits[0 * GMAX + blockIdx.x] = orc;
        ws.bits[1 * GMAX + blockIdx.x] = andc;
        ws.bits[2 * GMAX + blockIdx.x] = ora;
        ws.bits[3 * GMAX + blockIdx.x] = anda;
    }
}

// K5: stable compaction of the candidates (index order) and the first radix pass's histogram
__global__ __launch_bounds__(GT) void k_smp_compact(qmh_sample_args a) {
    constexpr int LT = 8;  // tiles one workgroup's output can span, counted in LDS
    __shared__ int pre_cnt[MAXCH];
    __shared__ uint32_t lh[LT * 256];
    __shared__ int wi[GT / 64];
    const Ws ws = ws_of(a);
    if (ws.ctl->nan) return;
    const int t = threadIdx.x, lane = t & 63, w = t >> 6, n = a.n;
    const bool pre = prefilter_on(a);
    const float cut = pre ? prefilter_cut(a) : 0.0f;
    const int J = chunk_j(n), ch = 64 * J, nch = (n + ch - 1) / ch;
    for (int k = t; k < nch; k += GT) pre_cnt[k] = ws.ccnt[k];
    for (int k = t; k < LT * 256; k += GT) lh[k] = 0;
    // key bits of all workgroups of K4
    uint32_t b4[4] = {0, 0, 0, 0};
    for (int k = t; k < (int)gridDim.x; k += GT) {
        b4[0] |= ws.bits[0 * GMAX + k];
        b4[1] |= ~ws.bits[1 * GMAX + k];
        b4[2] |= ws.bits[2 * GMAX + k];
        b4[3] |= ~ws.bits[3 * GMAX + k];
    }
    for (int k = 0; k < 4; k++) b4[k] = (uint32_t)block_or_i<GT>((int)b4[k], wi);
    __syncthreads();
    int nc;
    lds_exscan_i<GT>(pre_cnt, nch, wi, &nc);
    const bool all = nc == 0 || !pre;  // an empty prefilter falls back to every index
    if (all) nc = n;
    const int kk = (a.top_k > 0 && a.top_k < nc) ? a.top_k : nc;
    const uint32_t diff = all ? (b4[2] ^ ~b4[3]) : (b4[0] ^ ~b4[1]);
    int npass = 0, shift[4] = {0, 0, 0, 0};
    for (int s = 0; s < 32; s += 8)
        if ((diff >> s) & 255u) shift[npass++] = s;
    if (blockIdx.x == 0 && t == 0) {
        ws.ctl->nc = nc;
        ws.ctl->kk = kk;
        ws.ctl->npass = npass;
        for (int k = 0; k < 4; k++) ws.ctl->shift[k] = shift[k];
    }
    // this workgroup's candidates are the contiguous output range [o0, o1)
    const int c0 = blockIdx.x * (GT / 64), c1 = min(c0 + GT / 64, nch);
    const int o0 = all ? c0 * ch : pre_cnt[c0];
    const int o1 = all ? min(c1 * ch, n) : (c1 < nch ? pre_cnt[c1] : nc);
    const int tile0 = o0 / TILE;
    const bool in_lds = o1 <= o0 || (o1 - 1) / TILE - tile0 < LT;
    const int c = c0 + w;
    if (c < nch) {
        int off = all ? c * ch : pre_cnt[c];
        for (int k = 0; k < J; k++) {
            const int i = c * ch + k * 64 + lane;
            const float q = i < n ? a.p[i] : 0.0f;
            const bool cand = i < n && (all || q >= cut);
            const uint64_t m = __ballot(cand);
            if (cand) {
                const uint32_t key = prob_key(q);
                const int pos = off + lanes_below(m);
                a.key0[pos] = key;
                a.idx0[pos] = i;
                if (npass > 0) {
                    const uint32_t d = (key >> shift[0]) & 255u;
                    if (in_lds)
                        atomicAdd(&lh[(pos / TILE - tile0) * 256 + d], 1u);
                    else
                        atomicAdd(&ws.hist[(pos / TILE) * 256 + d], 1u);
                }
            }
            off += __popcll(m);
        }
    }
    __syncthreads();
    if (in_lds && npass > 0 && o1 > o0) {
        const int ntl = (o1 - 1) / TILE - tile0 + 1;
        for (int k = t; k < ntl * 256; k += GT)
            if (lh[k]) atomicAdd(&ws.hist[tile0 * 256 + k], lh[k]);
    }
}

// K6: radix pass p over tile blockIdx of the current array, stable, digits ranked per wave by
// ballots; the next pass's histogram is counted at the destination
__global__ __launch_bounds__(GT) void k_smp_pass(qmh_sample_args a, int p) {
    __shared__ uint32_t base[256];
    __shared__ uint32_t wc[GT / 64][256];
    __shared__ int wi[GT / 64];
    const Ws ws = ws_of(a);
    if (ws.ctl->nan || p >= ws.ctl->npass) return;
    const int nc = ws.ctl->nc, nt = (nc + TILE - 1) / TILE, tile = blockIdx.x;
    if (tile >= nt) return;
    const int t = threadIdx.x, lane = t & 63, w = t >> 6;
    const int ntm = ntile_max(a.n), npass = ws.ctl->npass, sft = ws.ctl->shift[p];
    const uint32_t *hist = ws.hist + (size_t)p * ntm * 256;
    uint32_t *hnext = p + 1 < npass ? ws.hist + (size_t)(p + 1) * ntm * 256 : nullptr;
    const int nsft = p + 1 < npass ? ws.ctl->shift[p + 1] : 0;
    const uint32_t *ks = (p & 1) ? a.key1 : a.key0;
    const int32_t *is = (p & 1) ? a.idx1 : a.idx0;
    uint32_t *kd = (p & 1) ? a.key0 : a.key1;
    int32_t *id = (p & 1) ? a.idx0 : a.idx1;
    // the wave's 4 rows of 64, loaded once, with the histogram column of digit t
    const int r0 = tile * TILE + w * 256;
    uint32_t key[4];
    int32_t ix[4];
#pragma unroll
    for (int r = 0; r < 4; r++) {
        const int i = r0 + r * 64 + lane;
        key[r] = i < nc ? ks[i] : 0u;
        ix[r] = i < nc ? is[i] : 0;
    }
    {
        // digit d = thread t: elements of digit d before this tile, then of smaller digits
        uint32_t tot = 0, pre = 0;
        for (int t0 = 0; t0 < nt; t0 += 32) {  // 32 loads in flight
            uint32_t h[32];
#pragma unroll
            for (int k = 0; k < 32; k++) h[k] = t0 + k < nt ? hist[(t0 + k) * 256 + t] : 0u;
#pragma unroll
            for (int k = 0; k < 32; k++) {
                tot += h[k];
                pre += t0 + k < tile ? h[k] : 0u;
            }
        }
        int dummy;
        base[t] = (uint32_t)block_exscan_i<GT>((int)tot, wi, &dummy) + pre;
        for (int k = 0; k < GT / 64; k++) wc[k][t] = 0;
    }
    __syncthreads();
#pragma unroll
    for (int r = 0; r < 4; r++) {
        const bool valid = r0 + r * 64 + lane < nc;
        const uint32_t d = (key[r] >> sft) & 255u;
        const uint64_t peers = digit_peers(d, valid);
        if (valid && lanes_below(peers) == 0) wc[w][d] += (uint32_t)__popcll(peers);
    }
    __syncthreads();
    {
        uint32_t run = base[t];
        for (int k = 0; k < GT / 64; k++) {
            const uint32_t c = wc[k][t];
            wc[k][t] = run;
            run += c;
        }
    }
    __syncthreads();
    for (int r = 0; r < 4; r++) {
        const bool valid = r0 + r * 64 + lane < nc;
        const uint32_t d = (key[r] >> sft) & 255u;
        const uint64_t peers = digit_peers(d, valid);
        const uint32_t b = valid ? wc[w][d] : 0u;
        const int rank = lanes_below(peers);
        if (valid) {
            const uint32_t pos = b + (uint32_t)rank;
            kd[pos] = key[r];
            id[pos] = ix[r];
            if (rank == 0) wc[w][d] = b + (uint32_t)__popcll(peers);
            if (hnext) atomicAdd(&hnext[(pos / TILE) * 256 + ((key[r] >> nsft) & 255u)], 1u);
        }
    }
}

// K7: approximate chunk sums of the nucleus (sorted probabilities)
__global__ __launch_bounds__(GT) void k_smp_nsum(qmh_sample_args a) {
    const Ws ws = ws_of(a);
    if (ws.ctl->nan) return;
    const int kk = ws.ctl->kk, J = chunk_j(kk), nch = (kk + 64 * J - 1) / (64 * J);
    const int c = blockIdx.x * (GT / 64) + (threadIdx.x >> 6);
    if (c >= nch) return;
    const uint32_t *kv = sorted_keys(a, ws.ctl);
    const double s = wave_chunk_sum([&](int i) { return key_prob(kv[i]); }, c, J, kk);
    if ((threadIdx.x & 63) == 0) ws.csum[c] = s;
}

// K9: the nucleus sum, the searches, the draw and the token (src/sampler.c:88-105)
__global__ __launch_bounds__(NTF) void k_smp_draw(qmh_sample_args a) {
    __shared__ ExSums x;
    const Ws ws = ws_of(a);
    Ctl *ctl = ws.ctl;
    const int t = threadIdx.x;
    if (ctl->nan) {  // the reference's sum is NaN and its heap returns index 0
        __syncthreads();  // every thread has read the flag
        if (t == 0) {
            uint64_t st = *a.rng;
            rng_uniform(&st);
            *a.rng = st;
            emit(a, 0);
            ctl->nan = 0;
            if (a.diag) {
                a.diag[0] = __builtin_nan("");
                a.diag[1] = 0;
            }
        }
        return;
    }
    const int kk = ctl->kk;
    const uint32_t *kv = sorted_keys(a, ctl);
    auto getq = [&](int i) { return key_prob(kv[i]); };
    fin_sums(getq, kk, ws, x, 2, a.force_serial != 0);
    const int ch = 64 * chunk_j(kk);
    const double tp = (double)a.top_p;
    const int first = exact_first<NTF>(getq, ch, kk, x, [&](double s) { return s >= tp; });
    const int m = first == NONE ? kk : first + 1;
    const double mass = exact_prefix(getq, ch, m, x);
    if (t == 0) {
        uint64_t st = *a.rng;
        const float u01 = rng_uniform(&st);  // one draw per non-greedy call (src/sampler.c:100)
        *a.rng = st;
        x.csum[0] = (double)u01 * mass;
    }
    __syncthreads();
    const double u = x.csum[0];
    const int hit = exact_first<NTF>(getq, ch, m, x, [&](double s) { return u < s; });
    if (t == 0) {
        emit(a, sorted_idx(a, ctl)[hit == NONE ? m - 1 : hit]);
        if (a.diag) {
            a.diag[0] = ctl->S;
            a.diag[1] = (double)(ctl->status | x.status);
            a.diag[2] = (double)ctl->nx_sum;
            a.diag[3] = (double)ctl->nc;
            a.diag[4] = (double)kk;
            a.diag[5] = (double)m;
            a.diag[6] = (double)x.nx;
            a.diag[7] = mass;
        }
    }
}

// zeroes the control block of a workspace whose previous contents are unknown (the static scratch)
__global__ void k_smp_clear(qmh_sample_args a) {
    uint32_t *c = (uint32_t *)a.ws;
    for (int i = threadIdx.x; i < (int)(sizeof(Ctl) / 4); i += blockDim.x) c[i] = 0;
}

// ---------------------------------------------------------------- static scratch
//
// The scratch of qmh_sample_noalloc: the probabilities, the two key and two index buffers of the
// radix sort, and the grid path's workspace, for vocabularies up to QMH_SAMPLE_NOALLOC_MAX_VOCAB.
// One copy per GPU, held until the process ends; every call on a GPU shares it.
constexpr size_t SCR_N = QMH_SAMPLE_NOALLOC_MAX_VOCAB;
constexpr size_t SCR_ARR = ws_align(SCR_N * 4);  // one [n] array of 4-byte elements
constexpr size_t SCR_BYTES = 5 * SCR_ARR + ws_align(ws_bytes((int)SCR_N));
static_assert(SCR_BYTES == QMH_SAMPLE_NOALLOC_BYTES, "scratch size stated in qmh_launch.h");

}  // namespace

static __device__ __align__(256) uint8_t scratch[SCR_BYTES];

// device address of the scratch on each device, looked up once per device with it current
#define QMH_MAX_DEVICES 64
static void *g_scratch_ptr[QMH_MAX_DEVICES];
static std::mutex g_scratch_mu;

extern "C" int qmh_sample_scratch(void **ptr) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return (int)e;
    if (dev < 0 || dev >= QMH_MAX_DEVICES) return (int)hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void *p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return (int)e;
        g_scratch_ptr[dev] = p;
    }
    *ptr = g_scratch_ptr[dev];
    return 0;
}

// the buffers of qmh_sample_args inside the scratch at base (a device address); the grid path's
// control block is cleared by a fill kernel on the stream first
extern "C" int qmh_launch_sample_scratch(qmh_sample_args *a, void *base, void *stream) {
    if (a->n < 1 || (size_t)a->n > SCR_N) return (int)hipErrorInvalidValue;
    uint8_t *b = (uint8_t *)base;
    a->p = (float *)b;
    a->key0 = (uint32_t *)(b + SCR_ARR);
    a->key1 = (uint32_t *)(b + 2 * SCR_ARR);
    a->idx0 = (int32_t *)(b + 3 * SCR_ARR);
    a->idx1 = (int32_t *)(b + 4 * SCR_ARR);
    a->ws = b + 5 * SCR_ARR;
    if (a->n > SMALL_N) {
        hipLaunchKernelGGL(k_smp_clear, dim3(1), dim3(64), 0, (hipStream_t)stream, *a);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return (int)e;
    }
    return qmh_launch_sample(a, stream);
}

extern "C" size_t qmh_sample_ws_bytes(int n) { return n > SMALL_N ? ws_bytes(n) : 0; }

extern "C" int qmh_launch_sample(const qmh_sample_args *a, void *stream) {
    hipStream_t s = (hipStream_t)stream;
    if (a->n <= SMALL_N) {
        hipLaunchKernelGGL(k_sample, dim3(1), dim3(NT1), 0, s, *a);
        return (int)hipGetLastError();
    }
    if (!a->ws) return (int)hipErrorInvalidValue;
    const int J = max(1, (a->n + 64 * MAXCH - 1) / (64 * MAXCH)), nch = (a->n + 64 * J - 1) / (64 * J);
    const dim3 g((nch + GT / 64 - 1) / (GT / 64)), b(GT), one(1), bf(NTF);
    hipLaunchKernelGGL(k_smp_exp, g, b, 0, s, *a);
    hipLaunchKernelGGL(k_smp_xfer<false>, g, b, 0, s, *a);
    hipLaunchKernelGGL(k_smp_norm, one, bf, 0, s, *a);
    hipLaunchKernelGGL(k_smp_prob, g, b, 0, s, *a);
    hipLaunchKernelGGL(k_smp_compact, g, b, 0, s, *a);
    for (int p = 0; p < 4; p++) hipLaunchKernelGGL(k_smp_pass, dim3(ntile_max(a->n)), b, 0, s, *a, p);
    hipLaunchKernelGGL(k_smp_nsum, g, b, 0, s, *a);
    hipLaunchKernelGGL(k_smp_xfer<true>, g, b, 0, s, *a);
    hipLaunchKernelGGL(k_smp_draw, one, bf, 0, s, *a);
    return (int)hipGetLastError();
}
