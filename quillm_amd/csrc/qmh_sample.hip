// gfx950 sampler: the reference's qm_sample (src/sampler.c:50-106) as one 1024-thread workgroup,
// token for token and rng state for rng state.
//
// The reference's result hangs on two serial double accumulations of floats: the normaliser
// sum += p[i] in index order (src/sampler.c:57-61), whose last bits decide every rounding of
// (float)(p[i] / sum), and the cumulative mass over the sorted candidates (src/sampler.c:89-104),
// which decides the nucleus and the drawn index. Both are computed here exactly, in parallel:
//
//   * thread t owns the chunk [t*C, t*C+C) and sums it approximately; a block scan gives every
//     chunk an approximate start a0 and end a1 (relative error below 2^-27 for n <= 2^24);
//   * while the serial sum s stays inside one binade [2^e, 2^(e+1)), adding v rounds v alone to a
//     multiple of ulp = 2^(e-52): s' = s + RNE(v), order-free, except at an exact tie, where
//     round-half-even looks at the parity of s/ulp. A chunk whose a0 and a1 lie in the same binade
//     with a margin (2^-26 relative) keeps the serial sum in it, and its effect on s is a function of
//     the incoming parity only: (increment, outgoing parity) for parity 0 and for parity 1;
//   * those functions compose associatively, so one segmented scan over chunks gives each chunk the
//     composition since the last chunk that could not be certified (a binade change, a margin miss,
//     or the first nonzero chunk); one wave replays the uncertified chunks serially, in order, from
//     their exact entry value (typically ~10 of 1024 chunks);
//   * every thread then knows the exact serial value at its chunk start and replays its own chunk
//     with the reference's own `s += v` when it needs per-element prefixes. Each chunk's replayed
//     end is checked against the next chunk's start (diag status bits).
//
// Candidates are sorted by (probability descending, index ascending) with a stable LSD radix sort
// on the probability bits (the heap of src/sampler.c:75-87 produces exactly this order: its less()
// is a total order when no probability is NaN). A NaN probability makes the reference's sum NaN,
// every probability NaN, and its heap then returns index 0 after drawing once: handled directly.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "qmh_device.h"
#include "qmh_launch.h"

namespace {

constexpr int NT = 1024, NW = NT / 64;
constexpr int NONE = 0x7fffffff;

struct SmpShared {
    union {
        uint32_t cnt[16 * NT];  // radix-sort counters, digit-major
        struct {
            long long i0[NT], i1[NT];  // chunk transfer: increment for incoming parity 0 / 1
            int ob[NT];                // bit0/bit1: outgoing parity for 0/1, bit2: chunk replayed serially
            int xlist[NT];             // replayed chunks in order
            double xin[NT], xout[NT];  // their exact entry / exit values
            double start[NT];          // every chunk's exact start (for the end-to-start check)
        } ex;
    };
    double wd[NW];
    int wi[NW];
    float wf[NW];
    double total, mass;
    int nx, status, mpos, tpos;
    uint32_t kor, kand;
};

// ---------------------------------------------------------------- block helpers (NT threads)

__device__ __forceinline__ int block_exscan_i(int v, int *wbuf, int *total) {
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
__device__ __forceinline__ double block_exscan_d(double v, double *wbuf) {
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

__device__ __forceinline__ int block_min_i(int v, int *wbuf) {
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

__device__ __forceinline__ float block_max_f(float v, float *wbuf) {
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

__device__ __forceinline__ int block_or_i(int v, int *wbuf) {
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

// ---------------------------------------------------------------- exact serial double sums

// binade exponent of a positive normal double
__device__ __forceinline__ int binade(double a) { return (int)((__double_as_longlong(a) >> 52) & 0x7ff) - 1023; }

// a (within 2^-27 relative of the serial value) certifies the serial value's binade e
__device__ __forceinline__ bool band_certified(double a, int e) {
    return a >= ldexp(1.0, e) * (1.0 + 0x1p-26) && a <= ldexp(1.0, e + 1) * (1.0 - 0x1p-26);
}

// a chunk's transfer (i0, i1, ob) applied to an exact serial value s (s = 0 only before the
// first nonzero chunk, where every certified chunk is all zeros)
__device__ __forceinline__ double xfer_apply(long long i0, long long i1, double s) {
    if (s == 0.0) return 0.0;
    const long long bits = __double_as_longlong(s);
    const long long inc = (bits & 1) ? i1 : i0;
    return s + (double)inc * ldexp(1.0, binade(s) - 52);
}

// (a then b); bit2 of ob marks a reset (a replayed chunk): the composition restarts after it
__device__ __forceinline__ void xfer_then(long long &a0, long long &a1, int &ao, long long b0, long long b1, int bo) {
    if (bo & 4) {
        a0 = b0;
        a1 = b1;
        ao = bo;
        return;
    }
    const int p0 = ao & 1, p1 = (ao >> 1) & 1;
    a0 += p0 ? b1 : b0;
    a1 += p1 ? b1 : b0;
    ao = (ao & 4) | ((bo >> p0) & 1) | (((bo >> p1) & 1) << 1);
}

// Exact serial prefix of s += (double)v[i] over i < len (v finite, >= 0, fetched by get(i)).
// Thread t owns [t*C, min(t*C+C, len)); returns the exact serial value at t*C. sh.total gets the
// exact final sum, sh.nx the number of chunks replayed serially; a replay that disagrees with the
// next chunk's computed start sets `bad` in sh.status (never expected).
template <class Get>
__device__ double exact_chunk_starts(const Get &get, int len, int C, SmpShared &sh, int bad) {
    const int t = threadIdx.x, lane = t & 63;
    const int lo = min(t * C, len), hi = min(lo + C, len);
    double loc = 0.0;
    for (int j = lo; j < hi; j++) loc += (double)get(j);
    const double a0 = block_exscan_d(loc, sh.wd), a1 = a0 + loc;
    // classify: certified (transfer function) or replayed
    bool replay = false;
    long long x0 = 0, x1 = 1;
    if (lo < hi && a1 != 0.0) {
        if (a0 == 0.0) {
            replay = true;
        } else {
            const int e = binade(a0);
            if (binade(a1) != e || !band_certified(a0, e) || !band_certified(a1, e)) {
                replay = true;
            } else {
                const double scale = ldexp(1.0, 52 - e);  // v / ulp, exact
                for (int j = lo; j < hi; j++) {
                    const double y = (double)get(j) * scale;
                    const double fl = floor(y);
                    const double fr = y - fl;
                    const long long a = (long long)fl;
                    if (fr == 0.5) {  // exact tie: round half to even on the running value
                        x0 += a;
                        x0 += x0 & 1;
                        x1 += a;
                        x1 += x1 & 1;
                    } else {
                        const long long r = a + (fr > 0.5 ? 1 : 0);
                        x0 += r;
                        x1 += r;
                    }
                }
            }
        }
    }
    int nx;
    const int xord = block_exscan_i(replay ? 1 : 0, sh.wi, &nx);
    if (replay) {
        sh.ex.xlist[xord] = t;
        sh.ex.i0[t] = 0;
        sh.ex.i1[t] = 0;
        sh.ex.ob[t] = 4 | 2;
    } else {
        sh.ex.i0[t] = x0;
        sh.ex.i1[t] = x1 - 1;
        sh.ex.ob[t] = (int)(x0 & 1) | ((int)(x1 & 1) << 1);
    }
    __syncthreads();
    if (t < 64) {
        // segmented exclusive scan of the 1024 transfers: lane l composes entries 16l .. 16l+15
        long long c0 = 0, c1 = 0;
        int co = 2;
        for (int k = 0; k < 16; k++) xfer_then(c0, c1, co, sh.ex.i0[16 * lane + k], sh.ex.i1[16 * lane + k],
                                               sh.ex.ob[16 * lane + k]);
        // inclusive wave scan of the lane aggregates, then shift to exclusive
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
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
        long long p0 = __shfl_up(c0, 1), p1 = __shfl_up(c1, 1);
        int po = __shfl_up(co, 1);
        if (lane == 0) {
            p0 = 0;
            p1 = 0;
            po = 2;
        }
        for (int k = 0; k < 16; k++) {
            const int i = 16 * lane + k;
            const long long e0 = sh.ex.i0[i], e1 = sh.ex.i1[i];
            const int eo = sh.ex.ob[i];
            sh.ex.i0[i] = p0;
            sh.ex.i1[i] = p1;
            sh.ex.ob[i] = (po & 3) | (eo & 4);  // keep the entry's own replay mark
            xfer_then(p0, p1, po, e0, e1, eo);
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");  // the wave reads other lanes' entries
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
        // serial walk over the replayed chunks, one wave: lanes fetch, the sum runs in order
        double s = 0.0;
        for (int k = 0; k < nx; k++) {
            const int x = __builtin_amdgcn_readfirstlane(sh.ex.xlist[k]);
            double cur = xfer_apply(sh.ex.i0[x], sh.ex.i1[x], s);
            const double sin = cur;
            const int xl = min(x * C, len), xh = min(xl + C, len);
            for (int b = xl; b < xh; b += 64) {
                const float v = b + lane < xh ? get(b + lane) : 0.0f;
                const int nb = min(64, xh - b);
                for (int q = 0; q < nb; q++)
                    cur += (double)__int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), q));
            }
            if (lane == 0) {
                sh.ex.xin[k] = sin;
                sh.ex.xout[k] = cur;
            }
            s = cur;
        }
        if (lane == 0) sh.nx = nx;
    }
    __syncthreads();
    const double start = replay ? sh.ex.xin[xord] : xfer_apply(sh.ex.i0[t], sh.ex.i1[t], xord > 0 ? sh.ex.xout[xord - 1] : 0.0);
    sh.ex.start[t] = start;
    __syncthreads();
    // replay the own chunk: its end must be the next chunk's start; the last chunk's end is the total
    double s = start;
    for (int j = lo; j < hi; j++) s += (double)get(j);
    const int last = len > 0 ? (len - 1) / C : 0;
    if (t == last) sh.total = s;
    if (t < last && s != sh.ex.start[t + 1]) atomicOr(&sh.status, bad);
    __syncthreads();
    return start;
}

// ---------------------------------------------------------------- the kernel

__device__ __forceinline__ float rng_uniform(uint64_t *state) {  // xorshift64* (src/sampler.c:18-25)
    uint64_t x = *state;
    x ^= x >> 12;
    x ^= x << 25;
    x ^= x >> 27;
    *state = x;
    return (float)((x * 0x2545F4914F6CDD1DULL) >> 40) / 16777216.0f;
}

__global__ __launch_bounds__(NT) void k_sample(qmh_sample_args a) {
    __shared__ SmpShared sh;
    const int t = threadIdx.x, n = a.n;
    if (t == 0) {
        sh.status = 0;
        sh.nx = 0;
    }
    // ---- exponentials (src/sampler.c:54-61): max by strict-greater scan from logits[0]
    float v = -__builtin_inff();
    for (int i = 1 + t; i < n; i += NT) {
        const float l = a.logits[i];
        v = l > v ? l : v;  // NaNs never win
    }
    v = block_max_f(v, sh.wf);
    const float l0 = a.logits[0];
    const float mx = v > l0 ? v : l0;  // a NaN logits[0] stays the maximum, as in the serial scan
    const float T = a.temperature;
    int nan = 0;
    for (int i = t; i < n; i += NT) {
        const float p = qmh_expf((a.logits[i] - mx) / T);
        nan |= p != p;
        a.p[i] = p;
    }
    nan = block_or_i(nan, sh.wi);
    float u01 = 0.0f;
    uint64_t st = 0;
    if (t == 0) {
        st = *a.rng;
        u01 = rng_uniform(&st);  // one draw per non-greedy call (src/sampler.c:100)
        *a.rng = st;
    }
    if (nan) {  // the reference's sum is NaN and its heap returns index 0
        if (t == 0) {
            if (a.out) *a.out = 0;
            if (a.tokpos) {
                a.tokpos[0] = 0;
                a.tokpos[1] += 1;
                const int step = a.tokpos[2];
                if (a.record && step >= 0 && step < a.record_cap) a.record[step] = 0;
                a.tokpos[2] = step + 1;
            }
            if (a.diag) {
                a.diag[0] = __builtin_nan("");
                a.diag[1] = 0;
            }
        }
        return;
    }
    __syncthreads();  // a.p visible to the workgroup
    // ---- exact serial normaliser, then probabilities (src/sampler.c:62)
    const int C = (n + NT - 1) / NT;
    const float *pv = a.p;
    exact_chunk_starts([&](int i) { return pv[i]; }, n, C, sh, 1);
    const double S = sh.total;
    const int nx_sum = sh.nx;
    // ---- candidates in index order (src/sampler.c:64-75), as (key, index) with
    //      key = bits(1.0f) - bits(q): ascending key = descending probability
    const bool pre = a.top_k == 0 && a.top_p < 1.0f && n > 1;
    const float cut = pre ? (1.0f - a.top_p) / (float)(n - 1) : 0.0f;
    const int lo = min(t * C, n), hi = min(lo + C, n);
    int cntc = 0;
    for (int j = lo; j < hi; j++) {
        const float q = (float)((double)a.p[j] / S);
        a.p[j] = q;
        cntc += (!pre || q >= cut) ? 1 : 0;
    }
    int nc;
    int off = block_exscan_i(cntc, sh.wi, &nc);
    const bool all = nc == 0 || !pre;
    if (all) {
        nc = n;
        off = lo;
    }
    uint32_t kor = 0, kand = 0xffffffffu;
    for (int j = lo; j < hi; j++) {
        const float q = a.p[j];
        if (all || q >= cut) {
            const uint32_t key = 0x3f800000u - __float_as_uint(q);
            a.key0[off] = key;
            a.idx0[off] = j;
            off++;
            kor |= key;
            kand &= key;
        }
    }
    // key bits that differ between candidates: a digit with none is the same for all, no pass
    const uint32_t any1 = (uint32_t)block_or_i((int)kor, sh.wi), all1 = ~(uint32_t)block_or_i((int)~kand, sh.wi);
    const uint32_t diff = any1 ^ all1;
    // ---- stable LSD radix sort of the candidates, 4-bit digits, passes over constant digits skipped
    uint32_t *ks = a.key0, *kd = a.key1;
    int32_t *is = a.idx0, *id = a.idx1;
    const int C3 = (nc + NT - 1) / NT;
    const int l3 = min(t * C3, nc), h3 = min(l3 + C3, nc);
    __syncthreads();
    for (int sft = 0; sft < 30; sft += 4) {
        if (((diff >> sft) & 15u) == 0) continue;
#pragma unroll
        for (int d = 0; d < 16; d++) sh.cnt[d * NT + t] = 0;
        for (int j = l3; j < h3; j++) sh.cnt[((ks[j] >> sft) & 15u) * NT + t]++;
        __syncthreads();
        uint32_t loc[16], tot = 0;
#pragma unroll
        for (int k = 0; k < 16; k++) {
            loc[k] = sh.cnt[16 * t + k];
            tot += loc[k];
        }
        int dummy;
        uint32_t run = (uint32_t)block_exscan_i((int)tot, sh.wi, &dummy);
#pragma unroll
        for (int k = 0; k < 16; k++) {
            sh.cnt[16 * t + k] = run;
            run += loc[k];
        }
        __syncthreads();
        for (int j = l3; j < h3; j++) {
            const uint32_t key = ks[j];
            const uint32_t pos = sh.cnt[((key >> sft) & 15u) * NT + t]++;
            kd[pos] = key;
            id[pos] = is[j];
        }
        __syncthreads();
        uint32_t *tk = ks;
        ks = kd;
        kd = tk;
        int32_t *ti = is;
        is = id;
        id = ti;
    }
    // ---- nucleus over the k best (src/sampler.c:88-99): exact serial cumulative mass
    const int kk = (a.top_k > 0 && a.top_k < nc) ? a.top_k : nc;
    const int C5 = (kk + NT - 1) / NT;
    const uint32_t *kv = ks;
    auto getq = [&](int i) { return __uint_as_float(0x3f800000u - kv[i]); };
    const double s0 = exact_chunk_starts(getq, kk, C5, sh, 2);
    const int l5 = min(t * C5, kk), h5 = min(l5 + C5, kk);
    const double tp = (double)a.top_p;
    int first = NONE;
    {
        double s = s0;
        for (int j = l5; j < h5; j++) {
            s += (double)getq(j);
            if (s >= tp) {
                first = j;
                break;
            }
        }
    }
    first = block_min_i(first, sh.wi);
    const int m = first == NONE ? kk : first + 1;
    if (t == (m - 1) / C5) {
        double s = s0;
        for (int j = l5; j < m; j++) s += (double)getq(j);
        sh.mass = s;
    }
    if (t == 0) sh.wd[0] = (double)u01;
    __syncthreads();
    const double mass = sh.mass;
    const double u = sh.wd[0] * mass;  // (double)u01 * mass (src/sampler.c:100)
    int hit = NONE;
    {
        double s = s0;
        for (int j = l5; j < min(h5, m); j++) {
            s += (double)getq(j);
            if (u < s) {
                hit = j;
                break;
            }
        }
    }
    hit = block_min_i(hit, sh.wi);
    if (t == 0) {
        const int tok = is[hit == NONE ? m - 1 : hit];
        if (a.out) *a.out = tok;
        if (a.tokpos) {
            a.tokpos[0] = tok;
            a.tokpos[1] += 1;
            const int step = a.tokpos[2];
            if (a.record && step >= 0 && step < a.record_cap) a.record[step] = tok;
            a.tokpos[2] = step + 1;
        }
        if (a.diag) {
            a.diag[0] = S;
            a.diag[1] = (double)sh.status;
            a.diag[2] = (double)nx_sum;
            a.diag[3] = (double)nc;
            a.diag[4] = (double)kk;
            a.diag[5] = (double)m;
            a.diag[6] = (double)sh.nx;
            a.diag[7] = mass;
        }
    }
}

}  // namespace

extern "C" int qmh_launch_sample(const qmh_sample_args *a, void *stream) {
    hipLaunchKernelGGL(k_sample, dim3(1), dim3(NT), 0, (hipStream_t)stream, *a);
    return (int)hipGetLastError();
}
