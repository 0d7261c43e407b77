// Device-side numerics shared by the gfx950 kernels.
//
// Everything here reproduces the reference's scalar CPU arithmetic bit for bit. The file is
// compiled with -ffp-contract=off, so a*b+c is two roundings, as in the reference (ISO C
// mode, no FMA); the only fused multiply-adds are the explicit fma() calls of qmh_expf and
// qmh_div127, parts of exact algorithms.
#pragma once

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#define QMH_WG 256  // threads per workgroup for the streaming kernels (4 wave64)

// a 16-byte-aligned float4 loaded non-temporally (data read once per step, e.g. the KV cache: it
// should not evict the code and the small vectors the next kernels read from L2)
typedef float qmh_v4f __attribute__((ext_vector_type(4)));
__device__ __forceinline__ float4 qmh_ld_nt4(const float *p) {
    const qmh_v4f v = __builtin_nontemporal_load((const qmh_v4f *)p);
    return make_float4(v.x, v.y, v.z, v.w);
}

// fp16 bits -> float. v_cvt_f32_f16 is exact for every finite half, subnormals included
// (fp16 denormals are on by default on gfx9); reference src/fp16.c:6-31.
__device__ __forceinline__ float qmh_h2f(uint16_t h) { return __half2float(__ushort_as_half(h)); }

// float -> fp16 bits, round to nearest even, as reference src/fp16.c:33-56 (NaN kept quiet with
// its top payload bits). Integer-only so the result does not depend on the MODE register, and
// branch-free: every case is computed and selected.
__device__ __forceinline__ uint16_t qmh_f2h(float f) {
    const uint32_t u = __float_as_uint(f);
    const uint32_t sign = (u >> 16) & 0x8000u, a = u & 0x7fffffffu;
    const int e = (int)(a >> 23) - 127;                   // unbiased exponent
    const uint32_t mant = (a & 0x7fffffu) | 0x800000u;
    int sh = e >= -14 ? 13 : 13 + (-14 - e);              // 13 (normal) .. subnormal shifts
    sh = sh < 25 ? sh : 25;                               // below 2^-25 everything rounds to 0
    uint32_t q = mant >> sh;
    const uint32_t rem = mant & ((1u << sh) - 1u), half = 1u << (sh - 1);
    q += (rem > half || (rem == half && (q & 1u))) ? 1u : 0u;
    // a normal q carries the implicit bit, so adding the biased exponent minus one both
    // places it and lets a rounding carry roll into the exponent (65520 -> inf)
    uint32_t r = e >= -14 ? (((uint32_t)(e + 14) << 10) + q) : q;
    r = e >= 16 ? 0x7c00u : r;                            // 2^16 and up (and inf) -> inf
    r = a > 0x7f800000u ? (0x7e00u | ((a >> 13) & 0x3ffu)) : r;
    return (uint16_t)(sign | r);
}

// m / 127.0f for m >= 0, correctly rounded without a division: q0 = m * fl(1/127), one FMA for
// the exact residual m - 127*q0 and one to correct q0. Checked equal to the IEEE quotient for
// every non-negative float except +inf, which is selected explicitly.
__device__ __forceinline__ float qmh_div127(float m) {
    const float r = 1.0f / 127.0f;
    const float q0 = m * r;
    const float q1 = __builtin_fmaf(__builtin_fmaf(-q0, 127.0f, m), r, q0);
    return m == __builtin_inff() ? m : q1;
}

// expf exactly as the host's glibc computes it (glibc >= 2.27 uses the ARM optimized-routines
// algorithm: x*32/ln2 = k + r, 2^(k/32) from a 32-entry table, a cubic for 2^(r/32), all in
// double, x86-64 FMA build). Checked equal to glibc expf for all 2^32 inputs on the host.
// The reference calls expf in softmax and SwiGLU (src/ops.c:107,131).
__constant__ static const uint64_t qmh_exp2_tab[32] = {
    0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,
    0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,
    0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
    0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,
    0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,
    0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
    0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,
    0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull};

// tab: the 32 entries of qmh_exp2_tab, wherever they are (a workgroup may keep a copy in LDS, to
// take the table lookup off global memory)
__device__ __forceinline__ float qmh_expf_t(float x, const uint64_t *tab) {
    uint32_t ux = __float_as_uint(x);
    uint32_t abstop = (ux >> 20) & 0x7ffu;
    if (abstop >= 0x42bu) {  // |x| >= 88, inf or nan
        if (ux == 0xff800000u) return 0.0f;
        if (abstop >= 0x7f8u) return x + x;
        if (x > 0x1.62e42ep6f) return __builtin_inff();
        if (x < -0x1.9fe368p6f) return 0.0f;
    }
    const double inv_ln2_n = 0x1.71547652b82fep+0 * 32.0, shift = 0x1.8p+52;
    const double c0 = 0x1.c6af84b912394p-5 / 32.0 / 32.0 / 32.0;
    const double c1 = 0x1.ebfce50fac4f3p-3 / 32.0 / 32.0;
    const double c2 = 0x1.62e42ff0c52d6p-1 / 32.0;
    double xd = (double)x;
    double kd = __builtin_fma(inv_ln2_n, xd, shift);
    uint64_t ki = (uint64_t)__double_as_longlong(kd);
    kd -= shift;
    double r = __builtin_fma(inv_ln2_n, xd, -kd);
    uint64_t t = tab[ki % 32] + (ki << 47);
    double s = __longlong_as_double((long long)t);
    double z = __builtin_fma(c0, r, c1);
    double r2 = r * r;
    double y = __builtin_fma(c2, r, 1.0);
    y = __builtin_fma(z, r2, y);
    y = y * s;
    return (float)y;
}
__device__ __forceinline__ float qmh_expf(float x) { return qmh_expf_t(x, qmh_exp2_tab); }
// --------------------------------------------------------------------------- reductions

template <int CTRL>
__device__ __forceinline__ int qmh_dpp(int v) {
    return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xf, 0xf, true);
}
#define QMH_DPP_QXOR1 0xb1      // quad_perm [1,0,3,2]
#define QMH_DPP_QXOR2 0x4e      // quad_perm [2,3,0,1]
#define QMH_DPP_HALF_MIRROR 0x141
#define QMH_DPP_MIRROR 0x140
template <int CTRL>
__device__ __forceinline__ double qmh_dpp_d(double v) {
    const int lo = qmh_dpp<CTRL>(__double2loint(v)), hi = qmh_dpp<CTRL>(__double2hiint(v));
    return __hiloint2double(hi, lo);
}
// The value of lane ^ 16 and of lane ^ 32, VALU only (gfx950's v_permlane16_swap / v_permlane32_swap
// with both operands v: lanes of the lower row/half get the upper's values in the second result,
// lanes of the upper in the first), instead of an LDS round trip through ds_bpermute.
__device__ __forceinline__ uint32_t qmh_xor16_u(uint32_t v) {
    const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
    return (threadIdx.x & 16) ? r[0] : r[1];
}
__device__ __forceinline__ uint32_t qmh_xor32_u(uint32_t v) {
    const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    return (threadIdx.x & 32) ? r[0] : r[1];
}
__device__ __forceinline__ double qmh_xor16_d(double v) {
    return __hiloint2double((int)qmh_xor16_u((uint32_t)__double2hiint(v)), (int)qmh_xor16_u((uint32_t)__double2loint(v)));
}
__device__ __forceinline__ double qmh_xor32_d(double v) {
    return __hiloint2double((int)qmh_xor32_u((uint32_t)__double2hiint(v)), (int)qmh_xor32_u((uint32_t)__double2loint(v)));
}
// max over the 64 lanes, every lane ending with it (DPP inside 16-lane rows, then the swaps)
__device__ __forceinline__ float qmh_wave_max(float v) {
    v = fmaxf(v, __int_as_float(qmh_dpp<QMH_DPP_QXOR1>(__float_as_int(v))));
    v = fmaxf(v, __int_as_float(qmh_dpp<QMH_DPP_QXOR2>(__float_as_int(v))));
    v = fmaxf(v, __int_as_float(qmh_dpp<QMH_DPP_HALF_MIRROR>(__float_as_int(v))));
    v = fmaxf(v, __int_as_float(qmh_dpp<QMH_DPP_MIRROR>(__float_as_int(v))));
    v = fmaxf(v, __uint_as_float(qmh_xor16_u(__float_as_uint(v))));
    return fmaxf(v, __uint_as_float(qmh_xor32_u(__float_as_uint(v))));
}
// sum over the 64 lanes (fixed order; all lanes get it): DPP within quads, 8- and 16-lane rows
// (the half-mirror / mirror pair each lane with one in the other half), then lane ^ 16, ^ 32
__device__ __forceinline__ double qmh_wave_sum_d(double v) {
    v += qmh_dpp_d<QMH_DPP_QXOR1>(v);
    v += qmh_dpp_d<QMH_DPP_QXOR2>(v);
    v += qmh_dpp_d<QMH_DPP_HALF_MIRROR>(v);
    v += qmh_dpp_d<QMH_DPP_MIRROR>(v);
    v += qmh_xor16_d(v);
    v += qmh_xor32_d(v);
    return v;
}

// Workgroup-wide sum of doubles (fixed tree: wave butterflies, then waves in order), result
// broadcast to all threads. buf: >= 16 doubles of LDS. Deterministic for a given blockDim.
__device__ __forceinline__ double qmh_block_sum_d(double v, double *buf) {
    v = qmh_wave_sum_d(v);
    const int w = threadIdx.x >> 6, nw = (blockDim.x + 63) >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) buf[w] = v;
    __syncthreads();
    double s = 0.0;
    for (int i = 0; i < nw; i++) s += buf[i];
    return s;
}

// The reference sums RMSNorm's squares (src/ops.c:95) and softmax's exponentials
// (src/ops.c:105-109) serially in double and uses each sum only through a float that is
// monotone in it: 1/sqrt(ss/n + eps) and 1/sum, each step correctly rounded. Here the sums are
// trees. Every summation order of n non-negative terms lies within gamma_{n-1}*S of the exact
// sum S, gamma_k = k*u/(1-k*u), u = 2^-53 (Higham, Accuracy and Stability of Numerical
// Algorithms, 2nd ed., section 4.2), so the serial sum lies in [s-d, s+d] for a tree's s and
// d = qmh_sum_slack(s, n) (2*gamma_{n-1}/(1-gamma_{n-1}) plus room for the rounding of d and
// s+-d). If the float of s-d equals that of s+d, monotonicity makes it the float of the serial
// sum too; otherwise (a fraction of about n * 7e-9 of the calls) the caller recomputes the sum
// serially in the reference's order. NaN and infinite sums always take the serial path.
__device__ __forceinline__ double qmh_sum_slack(double s, int n) { return s * ((double)n * 2.5 + 8.0) * 0x1p-53; }
__device__ __forceinline__ float qmh_rms_inv(double ss, int n, float eps) {
    return (float)(1.0 / sqrt(ss / (double)n + (double)eps));
}
__device__ __forceinline__ float qmh_recip_of_sum(double s) { return (float)(1.0 / s); }

// qmh_rms_inv for a sum known only to within the tree bound, without the correctly rounded
// double chain when the answer is clear. s: a tree sum of nterms squares; n: the row length.
// y = 1/sqrt(s/n + eps) from v_rsq_f64 (specified to 2^29 ulp, ~2^-23 relative) and two Newton
// steps (error 1.5*e^2 plus rounding, below 2^-50). For the serial sum S, |S - s| <= d with
// d/s = (nterms*2.5 + 8)*2^-53 (qmh_sum_slack), and the reference's double before its final
// rounding, fl(1/fl(sqrt(fl(fl(S/n) + eps)))), is within a relative d/(2s) + 3*2^-53 of
// 1/sqrt(S/n + eps), hence within M = y*(d/(2s) + 2^-46) of y. If y is farther than M from both
// midpoints between fl32(y) and its float neighbours, the reference rounds to fl32(y) too (never
// to a tie) and *out gets it; otherwise (relatively ~2^-16 of the inputs) it returns false and
// the caller takes the exact path.
__device__ __forceinline__ bool qmh_rms_inv_margin(double s, int n, int nterms, float eps, float *out) {
    const double x = s * (1.0 / (double)n) + (double)eps;
    double y = __builtin_amdgcn_rsq(x);
#pragma unroll
    for (int k = 0; k < 2; k++) {
        const double t = x * y;
        const double e = __builtin_fma(-t, y, 1.0);
        y = __builtin_fma(0.5 * y, e, y);
    }
    const float f = (float)y;
    const uint32_t fb = __float_as_uint(f);
    const double lo = 0.5 * ((double)f + (double)__uint_as_float(fb - 1u));
    const double hi = 0.5 * ((double)f + (double)__uint_as_float(fb + 1u));
    const double m = y * (((double)nterms * 2.5 + 8.0) * 0x1p-54 + 0x1p-46);
    *out = f;
    // finite, positive, normal: anything else (and every NaN comparison) goes the exact way
    return s >= 0.0 && y < 0x1p100 && fb > 0x00800000u && fb < 0x7f000000u && y - m > lo && y + m < hi;
}

__device__ __forceinline__ float qmh_block_max(float v, float *buf) {
    v = qmh_wave_max(v);
    const int w = threadIdx.x >> 6, nw = (blockDim.x + 63) >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) buf[w] = v;
    __syncthreads();
    float m = buf[0];
    for (int i = 1; i < nw; i++) m = fmaxf(m, buf[i]);
    return m;
}

// --------------------------------------------------------------------------- quantization

// One Q8_0 code: clamp(rint(v/dd), -127, 127), 0 when dd == 0 (reference src/quant.c:48-53).
// v/dd is the correctly rounded IEEE division (hipcc default), rintf is v_rndne_f32.
__device__ __forceinline__ int qmh_q8_code(float v, float dd) {
    if (dd == 0.0f) return 0;
    float r = rintf(v / dd);
    r = r < -127.0f ? -127.0f : r;
    r = r > 127.0f ? 127.0f : r;
    return (int)r;
}
// qmh_q8_code(v, dd) without a division in the common case. Let q = v/dd (real) and
// Q = fl(q), the correctly rounded quotient the reference rounds. rinv approximates 1/dd with
// relative error at most 2^-22 (the hardware reciprocal is specified to 1 ulp), so
// r = fl(v*rinv) = q(1+e1)(1+e2), |e1| <= 2^-22, |e2| <= 2^-24, and |Q - q| <= |q| 2^-24, giving
// |r - Q| <= |q| (2^-22 + 2^-23) (+ tiny). |v| <= amax and dd = fp32(fp16(amax/127)) >=
// (amax/127)/1.5 (fp16 subnormal rounding at worst), so |q| <= 190.5 and |r - Q| < 7e-5.
// Hence when r is more than 1e-4 from every rounding boundary k+1/2, rint(r) == rint(Q);
// otherwise (about 2 in 10^4 values, ties included) the exact division decides.
__device__ __forceinline__ float qmh_rcp(float x) { return __builtin_amdgcn_rcpf(x); }
__device__ __forceinline__ int qmh_q8_code_fast(float v, float dd, float rinv) {
    if (dd == 0.0f) return 0;
    const float r = v * rinv;
    float k = rintf(r);
    if (0.5f - fabsf(r - k) < 1e-4f) k = rintf(v / dd);
    k = k < -127.0f ? -127.0f : k;
    k = k > 127.0f ? 127.0f : k;
    return (int)k;
}
// the same for the 4 values of a lane, with one branch to the exact division for all of them
__device__ __forceinline__ void qmh_q8_codes4(const float *v, float dd, float rinv, int *q) {
    float k[4];
    bool slow = false;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const float r = v[j] * rinv;
        k[j] = rintf(r);
        slow |= 0.5f - fabsf(r - k[j]) < 1e-4f;
    }
    if (slow) {
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const float r = v[j] * rinv;
            if (0.5f - fabsf(r - rintf(r)) < 1e-4f) k[j] = rintf(v[j] / dd);
        }
    }
#pragma unroll
    for (int j = 0; j < 4; j++) {
        float c = k[j] < -127.0f ? -127.0f : k[j];
        c = c > 127.0f ? 127.0f : c;
        q[j] = dd == 0.0f ? 0 : (int)c;
    }
}

__device__ __forceinline__ int qmh_q4_code(float v, float dd) {
    if (dd == 0.0f) return 0;
    float r = rintf(v / dd);
    r = r < -8.0f ? -8.0f : r;
    r = r > 7.0f ? 7.0f : r;
    return (int)r;
}

// Reductions over 8 consecutive lanes with DPP (no LDS traffic): lane ^ 1 and lane ^ 2 inside
// each quad, then the row half-mirror (lane i <-> 7 - i of each 8-lane half row), which pairs
// every lane with one in the other quad. All 8 lanes end with the group's result.
// amax of a block spread over 8 consecutive lanes (4 values each): NaN never wins, like the
// reference's `a > amax` scan (src/quant.c:38-42).
__device__ __forceinline__ float qmh_amax8(float m) {
    float p = __int_as_float(qmh_dpp<QMH_DPP_QXOR1>(__float_as_int(m)));
    m = p > m ? p : m;
    p = __int_as_float(qmh_dpp<QMH_DPP_QXOR2>(__float_as_int(m)));
    m = p > m ? p : m;
    p = __int_as_float(qmh_dpp<QMH_DPP_HALF_MIRROR>(__float_as_int(m)));
    return p > m ? p : m;
}
// the same over the 4 lanes of a quad (lane ^ 1, then lane ^ 2)
__device__ __forceinline__ float qmh_amax4(float m) {
    float p = __int_as_float(qmh_dpp<QMH_DPP_QXOR1>(__float_as_int(m)));
    m = p > m ? p : m;
    p = __int_as_float(qmh_dpp<QMH_DPP_QXOR2>(__float_as_int(m)));
    return p > m ? p : m;
}
__device__ __forceinline__ int qmh_sum4(int v) {
    v += qmh_dpp<QMH_DPP_QXOR1>(v);
    return v + qmh_dpp<QMH_DPP_QXOR2>(v);
}
__device__ __forceinline__ int qmh_sum8(int v) {
    v += qmh_dpp<QMH_DPP_QXOR1>(v);
    v += qmh_dpp<QMH_DPP_QXOR2>(v);
    return v + qmh_dpp<QMH_DPP_HALF_MIRROR>(v);
}

// First index of the maximum of x[0..n) over the whole workgroup (src/sampler.c:27-32: `if (x[i] >
// x[best]) best = i` from best = 0, so a NaN at 0 wins and NaNs elsewhere are never chosen). Each
// thread walks its elements in increasing index order keeping the first strict maximum of the
// non-NaN values, with up to 8 loads in flight per round (VEC: 16-byte loads, x 16-byte aligned,
// so 32768 values take one round of 1024 threads); pairs then combine preferring the larger value,
// then the lower index, and a NaN x[0] overrides the result. The result is valid in thread 0.
template <bool VEC>
__device__ __forceinline__ int qmh_block_argmax(const float *__restrict__ x, int n, float *bv, int *bi) {
    float v = -__builtin_inff();
    int idx = 0x7fffffff;
    auto take = [&](float xv, int i) {
        if (xv == xv && (idx == 0x7fffffff || xv > v)) {
            v = xv;
            idx = i;
        }
    };
    const int nt = (int)blockDim.x;
    if (VEC) {
        const int n4 = n >> 2;
        const float4 *x4 = (const float4 *)x;
        for (int i0 = (int)threadIdx.x; i0 < n4; i0 += 8 * nt) {
            float4 xv[8];
#pragma unroll
            for (int k = 0; k < 8; k++) {
                const int i = i0 + k * nt;
                xv[k] = x4[i < n4 ? i : 0];
            }
#pragma unroll
            for (int k = 0; k < 8; k++) {
                const int i = i0 + k * nt;
                if (i < n4) {
                    take(xv[k].x, 4 * i);
                    take(xv[k].y, 4 * i + 1);
                    take(xv[k].z, 4 * i + 2);
                    take(xv[k].w, 4 * i + 3);
                }
            }
        }
        if ((int)threadIdx.x < (n & 3)) take(x[4 * n4 + (int)threadIdx.x], 4 * n4 + (int)threadIdx.x);
    } else {
        for (int i0 = (int)threadIdx.x; i0 < n; i0 += 8 * nt) {
            float xv[8];
#pragma unroll
            for (int k = 0; k < 8; k++) {
                const int i = i0 + k * nt;
                xv[k] = x[i < n ? i : 0];
            }
#pragma unroll
            for (int k = 0; k < 8; k++)
                if (i0 + k * nt < n) take(xv[k], i0 + k * nt);
        }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float ov = __shfl_xor(v, o);
        const int oi = __shfl_xor(idx, o);
        if (ov > v || (ov == v && oi < idx)) {
            v = ov;
            idx = oi;
        }
    }
    const int w = (int)threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) {
        bv[w] = v;
        bi[w] = idx;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int k = 1; k < nt >> 6; k++)
            if (bv[k] > v || (bv[k] == v && bi[k] < idx)) {
                v = bv[k];
                idx = bi[k];
            }
        if (idx == 0x7fffffff || x[0] != x[0]) idx = 0;  // all NaN, or NaN at 0
    }
    return idx;
}

// A serial chain over n terms in LDS (tp 16-byte aligned): y = y + t_i for i < n, in order. Sets of
// 32 terms are read as 8 float4s into three register sets, two sets ahead of the adds (the
// scheduling barriers hold the reads there). Measured on MI355X, one wave: a dependent add fed this
// way takes ~6.4 clocks, ~7.5 with one set ahead, ~12 with one 4-byte read per term (5.3 with the
// terms already in registers).
__device__ __forceinline__ float qmh_chain_lds(const float *tp, int n, float y) {
    const float4 *p4 = (const float4 *)tp;
    const int ns = n >> 5;  // whole sets
    float4 A[8], B[8], C[8];
    auto rd = [&](float4(&d)[8], int st) {
        st = st < ns ? st : ns - 1;  // past the last set: re-read it (no branch)
#pragma unroll
        for (int q = 0; q < 8; q++) d[q] = p4[8 * st + q];
    };
    auto add = [&](const float4(&d)[8]) {
#pragma unroll
        for (int q = 0; q < 8; q++) {
            y = y + d[q].x;
            y = y + d[q].y;
            y = y + d[q].z;
            y = y + d[q].w;
        }
    };
    if (ns > 0) {
        rd(A, 0);
        rd(B, 1);
        int st = 0;
        for (; st + 3 <= ns; st += 3) {
            rd(C, st + 2);
            __builtin_amdgcn_sched_barrier(0);
            add(A);
            __builtin_amdgcn_sched_barrier(0);
            rd(A, st + 3);
            __builtin_amdgcn_sched_barrier(0);
            add(B);
            __builtin_amdgcn_sched_barrier(0);
            rd(B, st + 4);
            __builtin_amdgcn_sched_barrier(0);
            add(C);
            __builtin_amdgcn_sched_barrier(0);
        }
        if (st < ns) add(A);
        if (st + 1 < ns) add(B);
    }
    for (int i = 8 * ns; i < (n >> 2); i++) {
        const float4 v = p4[i];
        y = y + v.x;
        y = y + v.y;
        y = y + v.z;
        y = y + v.w;
    }
    for (int i = n & ~3; i < n; i++) y = y + tp[i];
    return y;
}
