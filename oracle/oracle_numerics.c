/* CPU oracle, numerics part -- TEST INFRASTRUCTURE ONLY (see oracle.h).
 * Restates the reference's scalar arithmetic; each function cites what it follows. */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "oracle.h"

/* ---------------------------------------------------------------- fp16
 * IEEE binary16 <-> binary32, round-to-nearest-even (reference src/fp16.c:6-56). */

static uint32_t fbits(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    return u;
}
static float bitsf(uint32_t u) {
    float f;
    memcpy(&f, &u, 4);
    return f;
}

/* follows src/fp16.c:6-31. Subnormal halves are m * 2^-24, which is exact in float, so the
 * value is built by one exact multiply instead of a renormalising loop. */
float or_h2f(uint16_t h) {
    uint32_t sign = (uint32_t)(h >> 15) << 31;
    uint32_t e = (h >> 10) & 31u, m = h & 1023u;
    if (e == 31) return bitsf(sign | 0x7f800000u | (m << 13)); /* inf, NaN with payload */
    if (e != 0) return bitsf(sign | ((e + 112u) << 23) | (m << 13));
    if (m == 0) return bitsf(sign);
    return bitsf(sign | fbits((float)m * 0x1p-24f));
}

/* follows src/fp16.c:33-56: NaN keeps its top payload bits and is forced quiet; values at or
 * above 65520 become infinity; everything else is rounded to nearest-even, with one shift
 * count for normal (13) and subnormal (13 + how far below 2^-14) results. */
uint16_t or_f2h(float f) {
    uint32_t u = fbits(f);
    uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
    uint32_t a = u & 0x7fffffffu;
    if (a > 0x7f800000u) return (uint16_t)(sign | 0x7e00u | ((a >> 13) & 0x3ffu));
    int e = (int)(a >> 23) - 127; /* unbiased exponent of a normal float */
    if (e >= 16) return (uint16_t)(sign | 0x7c00u);
    if (e < -25) return sign; /* below 2^-25: rounds to zero (2^-25 itself ties to 0 below) */
    uint32_t mant = (a & 0x7fffffu) | 0x800000u;
    int shift = e >= -14 ? 13 : 13 + (-14 - e); /* 13..24 */
    uint32_t q = mant >> shift, rem = mant & ((1u << shift) - 1u), half = 1u << (shift - 1);
    if (rem > half || (rem == half && (q & 1u))) q++;
    /* normal: q holds the implicit bit (1024..2048); adding (e+14)<<10 both places the
     * exponent and lets a rounding carry bump it (65504+ -> 0x7c00). subnormal: q as is. */
    uint32_t r = e >= -14 ? (((uint32_t)(e + 14) << 10) + q) : q;
    return (uint16_t)(sign | r);
}

void or_f2h_array(const float *x, uint16_t *y, int64_t n) {
    for (int64_t i = 0; i < n; i++) y[i] = or_f2h(x[i]);
}
void or_h2f_array(const uint16_t *x, float *y, int64_t n) {
    for (int64_t i = 0; i < n; i++) y[i] = or_h2f(x[i]);
}

/* ---------------------------------------------------------------- quantization
 * Block formats (reference src/qm_base.h:17-29): Q8_0 = u16 fp16 scale + 32 x int8 (34 B);
 * Q4_0 = u16 fp16 scale + 16 bytes, element 2j in the low nibble of byte j, element 2j+1 in
 * the high nibble, value = d*(q-8) (18 B). Rows are zero-padded to whole blocks. */

int64_t or_nblocks(int64_t n) { return (n + 31) / 32; }

size_t or_row_bytes(int dtype, int64_t n) { /* src/quant.c:7-14 */
    if (dtype == OR_F32) return (size_t)n * 4;
    if (dtype == OR_Q8_0) return (size_t)or_nblocks(n) * 34;
    if (dtype == OR_Q4_0) return (size_t)or_nblocks(n) * 18;
    return 0;
}

/* one block's values with zero padding past n (src/quant.c:27-31) */
static void block_values(const float *x, int64_t n, int64_t b, float v[32]) {
    for (int i = 0; i < 32; i++) {
        int64_t k = b * 32 + i;
        v[i] = k < n ? x[k] : 0.0f;
    }
}

/* scale: d = amax/qmax in fp32, stored as fp16, used as fp32(fp16(d)) (src/quant.c:36-46) */
static float block_scale_h(const float v[32], float qmax, uint16_t *dh) {
    float amax = 0.0f;
    for (int i = 0; i < 32; i++) amax = fabsf(v[i]) > amax ? fabsf(v[i]) : amax;
    *dh = or_f2h(amax / qmax);
    return or_h2f(*dh);
}

/* q = clamp(rint(v/dd)) with dd == 0 -> 0 (src/quant.c:48-53) */
static int quant_code(float v, float dd, float lo, float hi) {
    if (dd == 0.0f) return 0;
    float r = rintf(v / dd);
    r = r < lo ? lo : r;
    r = r > hi ? hi : r;
    return (int)r;
}

static void put_u16(uint8_t *p, uint16_t v) {
    p[0] = (uint8_t)(v & 0xff);
    p[1] = (uint8_t)(v >> 8);
}
static uint16_t get_u16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }

void or_quantize_q8(const float *x, uint8_t *out, int64_t n) { /* src/quant.c:55-63 */
    for (int64_t b = 0; b < or_nblocks(n); b++) {
        float v[32];
        uint16_t dh;
        block_values(x, n, b, v);
        float dd = block_scale_h(v, 127.0f, &dh);
        uint8_t *blk = out + b * 34;
        put_u16(blk, dh);
        for (int i = 0; i < 32; i++) blk[2 + i] = (uint8_t)(int8_t)quant_code(v[i], dd, -127.0f, 127.0f);
    }
}

void or_quantize_q4(const float *x, uint8_t *out, int64_t n) { /* src/quant.c:72-85 */
    for (int64_t b = 0; b < or_nblocks(n); b++) {
        float v[32];
        uint16_t dh;
        block_values(x, n, b, v);
        float dd = block_scale_h(v, 7.0f, &dh);
        uint8_t *blk = out + b * 18;
        put_u16(blk, dh);
        for (int j = 0; j < 16; j++) {
            unsigned lo = (unsigned)(quant_code(v[2 * j], dd, -8.0f, 7.0f) + 8);
            unsigned hi = (unsigned)(quant_code(v[2 * j + 1], dd, -8.0f, 7.0f) + 8);
            blk[2 + j] = (uint8_t)(lo | (hi << 4));
        }
    }
}

void or_quantize_rows(int dtype, const float *x, uint8_t *out, int64_t rows, int64_t n) {
    size_t rb = or_row_bytes(dtype, n);
    for (int64_t r = 0; r < rows; r++) {
        if (dtype == OR_Q8_0) or_quantize_q8(x + r * n, out + r * rb, n);
        else if (dtype == OR_Q4_0) or_quantize_q4(x + r * n, out + r * rb, n);
        else memcpy(out + r * rb, x + r * n, rb);
    }
}

/* dequantize / copy a row to f32: d*q, exact in fp32 (src/quant.c:65-101) */
void or_row_to_f32(int dtype, const void *row, float *y, int64_t n) {
    const uint8_t *p = row;
    if (dtype == OR_F32) {
        memcpy(y, row, (size_t)n * 4);
        return;
    }
    for (int64_t i = 0; i < n; i++) {
        int64_t b = i / 32, k = i % 32;
        if (dtype == OR_Q8_0) {
            const uint8_t *blk = p + b * 34;
            y[i] = or_h2f(get_u16(blk)) * (float)(int8_t)blk[2 + k];
        } else {
            const uint8_t *blk = p + b * 18;
            uint8_t byte = blk[2 + k / 2];
            int q = (k & 1) ? (byte >> 4) : (byte & 15);
            y[i] = or_h2f(get_u16(blk)) * (float)(q - 8);
        }
    }
}

/* ---------------------------------------------------------------- dots (scalar order)
 * src/kernels_scalar.c:6-34: dot_f32 is one serial fp32 sum of products; the quantized dots
 * form an exact int32 per-block dot, then add (float)acc * (d_w*d_x) serially over blocks.
 * Every sum starts from +0.0f. */

float or_dot_f32(const float *a, const float *b, int64_t n) {
    float s = 0.0f;
    for (int64_t i = 0; i < n; i++) s = s + a[i] * b[i];
    return s;
}

float or_dot_q8(const uint8_t *w, const uint8_t *x, int64_t nb) {
    float s = 0.0f;
    for (int64_t b = 0; b < nb; b++) {
        const uint8_t *wb = w + b * 34, *xb = x + b * 34;
        int32_t acc = 0;
        for (int i = 0; i < 32; i++) acc += (int32_t)(int8_t)wb[2 + i] * (int32_t)(int8_t)xb[2 + i];
        float d = or_h2f(get_u16(wb)) * or_h2f(get_u16(xb));
        s = s + (float)acc * d;
    }
    return s;
}

float or_dot_q4(const uint8_t *w, const uint8_t *x, int64_t nb) {
    float s = 0.0f;
    for (int64_t b = 0; b < nb; b++) {
        const uint8_t *wb = w + b * 18, *xb = x + b * 34;
        int32_t acc = 0;
        for (int i = 0; i < 32; i++) {
            int q = ((wb[2 + i / 2] >> ((i & 1) * 4)) & 15) - 8;
            acc += q * (int32_t)(int8_t)xb[2 + i];
        }
        float d = or_h2f(get_u16(wb)) * or_h2f(get_u16(xb));
        s = s + (float)acc * d;
    }
    return s;
}

/* gemm_nt in the scalar ISA's order (src/gemm_driver.h:7-28 with src/kernels_scalar.c:36-44):
 * the K axis is cut into panels of 256; inside a panel each C element is a serial fp32 sum
 * of products from +0; the panel sums are added to C (which starts at +0) in panel order.
 * The 64-column and 4x4 tiling only decide who computes an element, not how, because the
 * edge path (dot_f32 over the panel) rounds exactly like the micro-tile. */
void or_gemm_nt(const float *A, const float *B, float *C, int64_t M, int64_t N, int64_t K, int64_t lda,
                int64_t ldb, int64_t ldc) {
    const int64_t KC = 256; /* QM_GEMM_KC, reference src/kernels.h:37 */
    for (int64_t i = 0; i < M; i++)
        for (int64_t j = 0; j < N; j++) {
            float c = 0.0f;
            for (int64_t k0 = 0; k0 < K; k0 += KC) {
                int64_t k1 = k0 + KC < K ? k0 + KC : K;
                float acc = 0.0f;
                for (int64_t k = k0; k < k1; k++) acc = acc + A[i * lda + k] * B[j * ldb + k];
                c = c + acc;
            }
            C[i * ldc + j] = c;
        }
}

/* src/ops.c:36-61: quantize x once (quantized W), then one dot per row */
void or_matvec(int dtype, const void *W, int64_t rows, int64_t cols, const float *x, float *y, uint8_t *xq) {
    const uint8_t *base = W;
    size_t rb = or_row_bytes(dtype, cols);
    int64_t nb = or_nblocks(cols);
    if (dtype != OR_F32) or_quantize_q8(x, xq, cols);
    for (int64_t r = 0; r < rows; r++) {
        const uint8_t *row = base + (size_t)r * rb;
        if (dtype == OR_F32) y[r] = or_dot_f32((const float *)(const void *)row, x, cols);
        else if (dtype == OR_Q8_0) y[r] = or_dot_q8(row, xq, nb);
        else y[r] = or_dot_q4(row, xq, nb);
    }
}

/* ---------------------------------------------------------------- elementwise (src/ops.c:93-133) */

/* sum of squares in double, serial; one fp32 scale; out = (x*inv)*w */
void or_rmsnorm(float *out, const float *x, const float *w, int64_t n, float eps) {
    double ss = 0.0;
    for (int64_t i = 0; i < n; i++) ss = ss + (double)x[i] * (double)x[i];
    float inv = (float)(1.0 / sqrt(ss / (double)n + (double)eps));
    for (int64_t i = 0; i < n; i++) out[i] = x[i] * inv * w[i];
}

/* max, expf(x - max), serial double sum, x *= (float)(1/sum) */
void or_softmax(float *x, int64_t n) {
    if (n <= 0) return;
    float mx = x[0];
    for (int64_t i = 1; i < n; i++) mx = x[i] > mx ? x[i] : mx;
    double sum = 0.0;
    for (int64_t i = 0; i < n; i++) {
        x[i] = expf(x[i] - mx);
        sum = sum + (double)x[i];
    }
    float inv = (float)(1.0 / sum);
    for (int64_t i = 0; i < n; i++) x[i] = x[i] * inv;
}

/* GPT-J style interleaved pairs; angle pos*theta^(-2i/hd) in double, cos/sin rounded to fp32 */
void or_rope(float *v, int64_t n_heads, int64_t head_dim, int64_t pos, float theta) {
    for (int64_t i = 0; i < head_dim / 2; i++) {
        double ang = (double)pos * pow((double)theta, -2.0 * (double)i / (double)head_dim);
        float c = (float)cos(ang), s = (float)sin(ang);
        for (int64_t h = 0; h < n_heads; h++) {
            float *p = v + h * head_dim + 2 * i;
            float x0 = p[0], x1 = p[1];
            p[0] = x0 * c - x1 * s;
            p[1] = x0 * s + x1 * c;
        }
    }
}

void or_swiglu(float *gate, const float *up, int64_t n) {
    for (int64_t i = 0; i < n; i++) gate[i] = gate[i] / (1.0f + expf(-gate[i])) * up[i];
}

/* first index of the maximum (reference src/sampler.c:27-32) */
int32_t or_argmax(const float *x, int32_t n) {
    int32_t best = 0;
    for (int32_t i = 1; i < n; i++)
        if (x[i] > x[best]) best = i;
    return best;
}

/* ---- sampler (reference src/sampler.c) ----
 *
 * Restated from the algorithm's definition rather than its heap: the reference keeps a size-k
 * min-heap under less(a,b) = p[a] < p[b] || (p[a] == p[b] && a > b) and heap-sorts it
 * (src/sampler.c:34-87). Without NaNs that order is total on distinct indices, so the heap's
 * output is exactly the k largest candidates sorted by (probability descending, index
 * ascending), which is what a comparison sort with that key yields here. With a NaN
 * probability the reference's serial double sum is NaN, every probability becomes NaN, less()
 * is always false, the heap never moves and the first heap-sort swap parks index 0 at position
 * k-1, which is returned (cum and u are NaN, so no earlier return): token 0. */
void or_sampler_init(or_sampler *s, int32_t n_vocab, float temperature, int top_k, float top_p, uint64_t seed) {
    /* parameter normalisation of src/sampler.c:8-12 */
    s->temperature = temperature < 0 ? 0 : temperature;
    s->top_k = top_k < 0 ? 0 : top_k;
    s->top_p = (top_p <= 0 || top_p > 1) ? 1.0f : top_p;
    s->rng = seed ? seed : 0x9e3779b97f4a7c15ULL;
    s->n_vocab = n_vocab;
}

/* xorshift64* (src/sampler.c:18-25): 24 high bits of the scrambled state over 2^24 */
float or_rng_uniform(uint64_t *state) {
    uint64_t x = *state;
    x ^= x >> 12;
    x ^= x << 25;
    x ^= x >> 27;
    *state = x;
    const uint64_t top24 = (x * 0x2545F4914F6CDD1DULL) >> 40;
    return (float)top24 / 16777216.0f;
}

static const float *g_sort_q;
static int cmp_desc(const void *pa, const void *pb) {
    const int32_t a = *(const int32_t *)pa, b = *(const int32_t *)pb;
    const float qa = g_sort_q[a], qb = g_sort_q[b];
    if (qa != qb) return qa > qb ? -1 : 1;
    return a < b ? -1 : (a > b);
}

int32_t or_sample(or_sampler *s, const float *logits, float *q, int32_t *order, double *sum_out) {
    const int32_t n = s->n_vocab;
    if (s->temperature == 0.0f || s->top_k == 1) return or_argmax(logits, n); /* src/sampler.c:52 */
    /* max by a strict-greater scan from logits[0] (src/sampler.c:54-56) */
    float mx = logits[0];
    for (int32_t i = 1; i < n; i++)
        if (logits[i] > mx) mx = logits[i];
    /* exponentials as floats, summed in index order in double (src/sampler.c:57-61) */
    double sum = 0;
    for (int32_t i = 0; i < n; i++) {
        q[i] = expf((logits[i] - mx) / s->temperature);
        sum += q[i];
    }
    if (sum_out) *sum_out = sum;
    for (int32_t i = 0; i < n; i++) q[i] = (float)(q[i] / sum); /* src/sampler.c:62 */
    const float u01 = or_rng_uniform(&s->rng);                 /* drawn once per non-greedy call */
    if (sum != sum) return 0;                                   /* NaN: see the header comment */
    /* candidates (src/sampler.c:64-75): the top-p prefilter, or every index */
    int32_t nc = 0;
    if (s->top_k == 0 && s->top_p < 1.0f && n > 1) {
        const float cut = (1.0f - s->top_p) / (float)(n - 1);
        for (int32_t i = 0; i < n; i++)
            if (q[i] >= cut) order[nc++] = i;
    }
    if (nc == 0)
        for (int32_t i = 0; i < n; i++) order[nc++] = i;
    const int32_t k = (s->top_k > 0 && s->top_k < nc) ? s->top_k : nc;
    g_sort_q = q;
    qsort(order, (size_t)nc, sizeof(int32_t), cmp_desc);
    /* nucleus: the shortest prefix whose serial double sum reaches top_p (src/sampler.c:89-99) */
    double cum = 0;
    int32_t m = k;
    for (int32_t i = 0; i < k; i++) {
        cum += q[order[i]];
        if (cum >= s->top_p) {
            m = i + 1;
            break;
        }
    }
    double mass = 0;
    for (int32_t i = 0; i < m; i++) mass += q[order[i]];
    /* inverse-CDF draw over the nucleus (src/sampler.c:100-105) */
    const double u = (double)u01 * mass;
    double c = 0;
    for (int32_t i = 0; i < m; i++) {
        c += q[order[i]];
        if (u < c) return order[i];
    }
    return order[m - 1];
}
