// gfx950 small kernels of the quillm token loop: embedding, argmax, and the op-level
// numerics (fp16, quantization, RMSNorm, softmax, RoPE, SwiGLU, gemm_nt).
//
// Rounding contract: bit-identical to the reference's scalar CPU path (built with
// -ffp-contract=off). The double-precision sums of RMSNorm and softmax are trees whose float
// results are checked against the serial order's error bound (qmh_sum_slack), with a serial
// recomputation when the bound cannot decide them.
#include "qmh_device.h"
#include "qmh_launch.h"

#define QMH_Q8 2
#define QMH_Q4 3

// ============================================================================ embedding

// x = dequantised row `token` of tok_embd (src/model.c:162 -> src/quant.c:65-101)
__global__ void k_embed(const uint8_t *__restrict__ E, int dtype, int dim, int vocab, const int32_t *tok_ptr,
                        float *x, uint32_t *step_ctr) {
    if (step_ctr && blockIdx.x == 0 && threadIdx.x == 0) step_ctr[0] += 1u;
    const int tok = *tok_ptr;
    if (tok < 0 || tok >= vocab) return;  // stale token in device memory: read nothing
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < dim; i += gridDim.x * blockDim.x) {
        const int b = i >> 5, k = i & 31;
        float v;
        if (dtype == QMH_Q8) {
            const uint8_t *blk = E + ((size_t)tok * ((dim + 31) / 32) + b) * 34;
            v = qmh_h2f((uint16_t)(blk[0] | (blk[1] << 8))) * (float)(int8_t)blk[2 + k];
        } else if (dtype == QMH_Q4) {
            const uint8_t *blk = E + ((size_t)tok * ((dim + 31) / 32) + b) * 18;
            const uint8_t byte = blk[2 + (k >> 1)];
            const int q = (k & 1) ? (byte >> 4) : (byte & 15);
            v = qmh_h2f((uint16_t)(blk[0] | (blk[1] << 8))) * (float)(q - 8);
        } else {
            v = ((const float *)E)[(size_t)tok * dim + i];
        }
        x[i] = v;
    }
}

extern "C" int qmh_launch_embed(const uint8_t *tok_embd, int dtype, int dim, int vocab, const int32_t *tok_ptr,
                                float *x, uint32_t *step_ctr, void *stream) {
    hipLaunchKernelGGL(k_embed, dim3((dim + 255) / 256), dim3(256), 0, (hipStream_t)stream, tok_embd, dtype, dim,
                       vocab, tok_ptr, x, step_ctr);
    return (int)hipGetLastError();
}

// ============================================================================ argmax

// argmax over x[n] (qmh_block_argmax, one workgroup of 1024 threads; 16-byte loads when x is 16-byte
// aligned), with the decode loop's bookkeeping when tokpos != NULL: tokpos[0] = the token,
// tokpos[1] += 1, record[tokpos[2]] = it, tokpos[2] += 1
template <bool VEC>
__global__ __launch_bounds__(1024) void k_argmax(const float *__restrict__ x, int n, int32_t *out_idx,
                                                 int32_t *tokpos, int32_t *record, int record_cap) {
    __shared__ float bv[16];
    __shared__ int bi[16];
    const int idx = qmh_block_argmax<VEC>(x, n, bv, bi);
    if (threadIdx.x == 0) {
        if (out_idx) *out_idx = idx;
        if (tokpos) {
            tokpos[0] = idx;
            tokpos[1] += 1;
            const int step = tokpos[2];
            if (record && step >= 0 && step < record_cap) record[step] = idx;
            tokpos[2] = step + 1;
        }
    }
}

extern "C" int qmh_launch_argmax(const float *x, int n, int32_t *out_idx, int32_t *tokpos, int32_t *record,
                                 int record_cap, void *stream) {
    if (((uintptr_t)x & 15) == 0)
        hipLaunchKernelGGL(k_argmax<true>, dim3(1), dim3(1024), 0, (hipStream_t)stream, x, n, out_idx, tokpos,
                           record, record_cap);
    else
        hipLaunchKernelGGL(k_argmax<false>, dim3(1), dim3(1024), 0, (hipStream_t)stream, x, n, out_idx, tokpos,
                           record, record_cap);
    return (int)hipGetLastError();
}

// ============================================================================ elementwise

__global__ void k_swiglu(float *gate, const float *up, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
        const float g = gate[i];
        gate[i] = g / (1.0f + qmh_expf(-g)) * up[i];
    }
}

extern "C" int qmh_launch_swiglu(float *gate, const float *up, int64_t n, void *stream) {
    if (n <= 0) return 0;
    int64_t grid = (n + 255) / 256;
    grid = grid > 4096 ? 4096 : grid;
    hipLaunchKernelGGL(k_swiglu, dim3((unsigned)grid), dim3(256), 0, (hipStream_t)stream, gate, up, n);
    return (int)hipGetLastError();
}

__global__ void k_h2f(const uint16_t *h, float *f, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
        f[i] = qmh_h2f(h[i]);
}
__global__ void k_f2h(const float *f, uint16_t *h, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
        h[i] = qmh_f2h(f[i]);
}

static unsigned grid_for(int64_t n) {
    int64_t g = (n + 255) / 256;
    return (unsigned)(g < 1 ? 1 : (g > 8192 ? 8192 : g));
}

extern "C" int qmh_launch_h2f(const uint16_t *h, float *f, int64_t n, void *stream) {
    if (n <= 0) return 0;
    hipLaunchKernelGGL(k_h2f, dim3(grid_for(n)), dim3(256), 0, (hipStream_t)stream, h, f, n);
    return (int)hipGetLastError();
}
extern "C" int qmh_launch_f2h(const float *f, uint16_t *h, int64_t n, void *stream) {
    if (n <= 0) return 0;
    hipLaunchKernelGGL(k_f2h, dim3(grid_for(n)), dim3(256), 0, (hipStream_t)stream, f, h, n);
    return (int)hipGetLastError();
}

// rows x n -> reference-layout Q8_0 / Q4_0 rows (src/quant.c:55-85); 8 lanes per block
__global__ void k_quantize_rows(const float *__restrict__ x, uint8_t *__restrict__ y, int64_t rows, int64_t n,
                                int dtype) {
    const int64_t nb = (n + 31) / 32;
    const int sub = threadIdx.x & 7;
    const int64_t gb = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 3;  // global block id
    const bool on = gb < rows * nb;
    const int64_t row = on ? gb / nb : 0, b = on ? gb % nb : 0;
    float v[4], m = 0.0f;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const int64_t i = b * 32 + sub * 4 + k;
        v[k] = (on && i < n) ? x[row * n + i] : 0.0f;
        const float av = fabsf(v[k]);
        m = av > m ? av : m;
    }
    m = qmh_amax8(m);
    const uint16_t dh = qmh_f2h(dtype == QMH_Q4 ? m / 7.0f : qmh_div127(m));
    const float dd = qmh_h2f(dh);
    if (!on) return;
    if (dtype == QMH_Q4) {
        uint8_t *o = y + (row * nb + b) * 18;
        if (sub == 0) {
            o[0] = (uint8_t)(dh & 0xff);
            o[1] = (uint8_t)(dh >> 8);
        }
        for (int j = 0; j < 2; j++) {
            const int lo = qmh_q4_code(v[2 * j], dd) + 8, hi = qmh_q4_code(v[2 * j + 1], dd) + 8;
            o[2 + sub * 2 + j] = (uint8_t)(lo | (hi << 4));
        }
    } else {
        uint8_t *o = y + (row * nb + b) * 34;
        if (sub == 0) {
            o[0] = (uint8_t)(dh & 0xff);
            o[1] = (uint8_t)(dh >> 8);
        }
        // the matvec prologue's division-free path (same codes; pinned here by the op tests)
        int q[4];
        qmh_q8_codes4(v, dd, qmh_rcp(dd), q);
#pragma unroll
        for (int k = 0; k < 4; k++) o[2 + sub * 4 + k] = (uint8_t)(int8_t)q[k];
    }
}

extern "C" int qmh_launch_quantize_rows(const float *x, uint8_t *y, int64_t rows, int64_t n, int dtype, void *stream) {
    const int64_t blocks = rows * ((n + 31) / 32);
    if (blocks <= 0) return 0;
    const int64_t grid = (blocks * 8 + 255) / 256;
    hipLaunchKernelGGL(k_quantize_rows, dim3((unsigned)grid), dim3(256), 0, (hipStream_t)stream, x, y, rows, n, dtype);
    return (int)hipGetLastError();
}

__global__ void k_row_to_f32(const uint8_t *__restrict__ row, int dtype, float *y, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t b = i >> 5;
        const int k = (int)(i & 31);
        if (dtype == QMH_Q8) {
            const uint8_t *blk = row + b * 34;
            y[i] = qmh_h2f((uint16_t)(blk[0] | (blk[1] << 8))) * (float)(int8_t)blk[2 + k];
        } else if (dtype == QMH_Q4) {
            const uint8_t *blk = row + b * 18;
            const uint8_t byte = blk[2 + (k >> 1)];
            const int q = (k & 1) ? (byte >> 4) : (byte & 15);
            y[i] = qmh_h2f((uint16_t)(blk[0] | (blk[1] << 8))) * (float)(q - 8);
        } else {
            y[i] = ((const float *)row)[i];
        }
    }
}

extern "C" int qmh_launch_row_to_f32(const uint8_t *row, int dtype, float *y, int64_t n, void *stream) {
    if (n <= 0) return 0;
    hipLaunchKernelGGL(k_row_to_f32, dim3(grid_for(n)), dim3(256), 0, (hipStream_t)stream, row, dtype, y, n);
    return (int)hipGetLastError();
}

// RMSNorm (src/ops.c:93-98): one workgroup; double sum of squares as a tree, checked against
// the serial order's error bound (qmh_sum_slack), then out = (x*inv)*w.
__global__ __launch_bounds__(1024) void k_rmsnorm(float *out, const float *x, const float *w, int64_t n, float eps) {
    __shared__ double red[16];
    double ss = 0.0;
    for (int64_t i = threadIdx.x; i < n; i += blockDim.x) ss += (double)x[i] * (double)x[i];
    ss = qmh_block_sum_d(ss, red);
    const double d = qmh_sum_slack(ss, (int)n);
    float inv = qmh_rms_inv(ss - d, (int)n, eps);
    if (inv != qmh_rms_inv(ss + d, (int)n, eps)) {  // uniform; serial sum as the reference
        if (threadIdx.x == 0) {
            double s = 0.0;
            for (int64_t i = 0; i < n; i++) s += (double)x[i] * (double)x[i];
            red[8] = s;
        }
        __syncthreads();
        inv = qmh_rms_inv(red[8], (int)n, eps);
    }
    for (int64_t i = threadIdx.x; i < n; i += blockDim.x) out[i] = x[i] * inv * w[i];
}

extern "C" int qmh_launch_rmsnorm(float *out, const float *x, const float *w, int64_t n, float eps, void *stream) {
    hipLaunchKernelGGL(k_rmsnorm, dim3(1), dim3(1024), 0, (hipStream_t)stream, out, x, w, n, eps);
    return (int)hipGetLastError();
}

// softmax (src/ops.c:100-112), one workgroup
__global__ __launch_bounds__(1024) void k_softmax(float *x, int64_t n) {
    __shared__ double red[16];
    __shared__ float redf[16];
    float m = -__builtin_inff();
    for (int64_t i = threadIdx.x; i < n; i += blockDim.x) m = x[i] > m ? x[i] : m;
    m = qmh_block_max(m, redf);
    double sum = 0.0;
    for (int64_t i = threadIdx.x; i < n; i += blockDim.x) {
        const float e = qmh_expf(x[i] - m);
        x[i] = e;
        sum += (double)e;
    }
    sum = qmh_block_sum_d(sum, red);
    const double d = qmh_sum_slack(sum, (int)n);
    float inv = qmh_recip_of_sum(sum - d);
    if (inv != qmh_recip_of_sum(sum + d)) {  // uniform; serial sum as the reference
        if (threadIdx.x == 0) {
            double s = 0.0;
            for (int64_t i = 0; i < n; i++) s += (double)x[i];  // this thread's own writes and
            red[8] = s;                                        // the others', published by the
        }                                                      // tree sum's barriers
        __syncthreads();
        inv = qmh_recip_of_sum(red[8]);
    }
    for (int64_t i = threadIdx.x; i < n; i += blockDim.x) x[i] = x[i] * inv;
}

extern "C" int qmh_launch_softmax(float *x, int64_t n, void *stream) {
    if (n <= 0) return 0;
    hipLaunchKernelGGL(k_softmax, dim3(1), dim3(1024), 0, (hipStream_t)stream, x, n);
    return (int)hipGetLastError();
}

// RoPE (src/ops.c:114-126) with the (cos, sin) pairs of one position precomputed on the host
// with the reference's double formula
__global__ void k_rope(float *v, int64_t n_heads, int64_t hd, const float *cs) {
    const int64_t npairs = n_heads * (hd / 2);
    for (int64_t p = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; p < npairs; p += (int64_t)gridDim.x * blockDim.x) {
        const int64_t h = p / (hd / 2), i = p % (hd / 2);
        float *e = v + h * hd + 2 * i;
        const float c = cs[2 * i], s = cs[2 * i + 1], x0 = e[0], x1 = e[1];
        e[0] = x0 * c - x1 * s;
        e[1] = x0 * s + x1 * c;
    }
}

extern "C" int qmh_launch_rope(float *v, int64_t n_heads, int64_t head_dim, const float *table, int64_t pos,
                               void *stream) {
    const int64_t npairs = n_heads * (head_dim / 2);
    if (npairs <= 0) return 0;
    hipLaunchKernelGGL(k_rope, dim3(grid_for(npairs)), dim3(256), 0, (hipStream_t)stream, v, n_heads, head_dim,
                       table + (size_t)pos * (head_dim / 2) * 2);
    return (int)hipGetLastError();
}

// gemm_nt in the scalar ISA's order (src/gemm_driver.h:7-28): per element, K is cut into
// panels of 256 (QM_GEMM_KC, src/kernels.h:37); each panel is a serial fp32 sum from +0 (each
// product rounded alone, then added) and the panel sums are added to C (from +0) in order.
// A workgroup of 256 threads owns 32x32 outputs, each thread a 2x2 block (four chains). A and B
// pass through LDS in slices of GN_KS values of k, stored k-major ([k][row], rows padded to 34 so
// the transposing writes are conflict-free and the float2 reads aligned); per k a thread reads two
// float2 (its rows' A, its columns' B: the wave's four row pairs are broadcast reads) for four
// multiplies and four adds. The next slice's global loads are in flight while a slice is summed.
// Elements past M, N or K are staged as 0 and never added or stored.
#define QMH_GEMM_KC 256
#define GN_T 32   // outputs per workgroup side
#define GN_KS 128  // k per LDS slice (divides QMH_GEMM_KC; a multiple of 32)
#define GN_NQ (GN_KS / 32)  // float4 loads per thread per operand and slice
#define GN_LD 34  // LDS row stride (floats)
template <bool VEC>
__global__ __launch_bounds__(256) void k_gemm_nt(const float *__restrict__ A, const float *__restrict__ B,
                                                 float *__restrict__ C, int64_t M, int64_t N, int64_t K) {
    static_assert(QMH_GEMM_KC % GN_KS == 0 && GN_T * GN_KS == 4 * 256 * GN_NQ, "whole float4s per thread per slice");
    __shared__ __align__(16) float As[GN_KS][GN_LD], Bs[GN_KS][GN_LD];
    const int tid = threadIdx.x, r = tid >> 4, c = tid & 15;  // rows 2r, 2r+1; columns 2c, 2c+1
    const int64_t i0 = (int64_t)blockIdx.y * GN_T, j0 = (int64_t)blockIdx.x * GN_T;
    // staging: thread t loads row t/8 of the tile, k 32*q + 4*(t%8) .. +3 of the slice (q < GN_NQ),
    // for A and for B
    const int sr = tid >> 3, sk = 4 * (tid & 7);
    const float *ar = A + (i0 + sr < M ? i0 + sr : 0) * K, *br = B + (j0 + sr < N ? j0 + sr : 0) * K;
    const bool aon = i0 + sr < M, bon = j0 + sr < N;
    // no branches, and the values past M, N or K are zeroed only when the slice is stored, so the
    // loads stay in flight under the previous slice's sums (VEC: K % 4 == 0 and rows 16-byte
    // aligned, so a thread's 4 values are all in the row or all past K)
    float va[GN_NQ][4], vb[GN_NQ][4];
    auto fetch = [&](const float *row, int64_t k0, float (&v)[GN_NQ][4]) {
#pragma unroll
        for (int q = 0; q < GN_NQ; q++) {
            const int64_t k = k0 + 32 * q + sk;
            if (VEC) {
                const float4 f = *(const float4 *)(row + (k < K ? k : 0));
                v[q][0] = f.x, v[q][1] = f.y, v[q][2] = f.z, v[q][3] = f.w;
            } else {
#pragma unroll
                for (int j = 0; j < 4; j++) v[q][j] = row[k + j < K ? k + j : K - 1];
            }
        }
    };
    float c00 = 0.0f, c01 = 0.0f, c10 = 0.0f, c11 = 0.0f;
    float s00 = 0.0f, s01 = 0.0f, s10 = 0.0f, s11 = 0.0f;
    fetch(ar, 0, va);
    fetch(br, 0, vb);
    for (int64_t k0 = 0; k0 < K; k0 += GN_KS) {
        __syncthreads();  // the previous slice is consumed
#pragma unroll
        for (int q = 0; q < GN_NQ; q++)
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const bool in = k0 + 32 * q + sk + j < K;
                As[32 * q + sk + j][sr] = aon && in ? va[q][j] : 0.0f;
                Bs[32 * q + sk + j][sr] = bon && in ? vb[q][j] : 0.0f;
            }
        __syncthreads();
        if (k0 + GN_KS < K) {  // uniform: the next slice's loads under this slice's sums
            fetch(ar, k0 + GN_KS, va);
            fetch(br, k0 + GN_KS, vb);
        }
        const int kn = K - k0 < GN_KS ? (int)(K - k0) : GN_KS;
        if (kn == GN_KS) {
            // groups of 8 k from two register sets: group g+1's reads go out before group g's
            // sums (held there by the scheduling barriers)
            float2 xa[2][8], xb[2][8];
            auto rd = [&](int g, float2(&da)[8], float2(&db)[8]) {
#pragma unroll
                for (int q = 0; q < 8; q++) {
                    da[q] = *(const float2 *)&As[8 * g + q][2 * r];
                    db[q] = *(const float2 *)&Bs[8 * g + q][2 * c];
                }
            };
            auto sum = [&](const float2(&da)[8], const float2(&db)[8]) {
#pragma unroll
                for (int q = 0; q < 8; q++) {
                    s00 = s00 + da[q].x * db[q].x;
                    s01 = s01 + da[q].x * db[q].y;
                    s10 = s10 + da[q].y * db[q].x;
                    s11 = s11 + da[q].y * db[q].y;
                }
            };
            rd(0, xa[0], xb[0]);
#pragma unroll
            for (int g = 0; g < GN_KS / 8; g++) {
                if (g + 1 < GN_KS / 8) rd(g + 1, xa[(g + 1) & 1], xb[(g + 1) & 1]);
                __builtin_amdgcn_sched_barrier(0);
                sum(xa[g & 1], xb[g & 1]);
                __builtin_amdgcn_sched_barrier(0);
            }
        } else {
            for (int k = 0; k < kn; k++) {
                const float2 a2 = *(const float2 *)&As[k][2 * r], b2 = *(const float2 *)&Bs[k][2 * c];
                s00 = s00 + a2.x * b2.x;
                s01 = s01 + a2.x * b2.y;
                s10 = s10 + a2.y * b2.x;
                s11 = s11 + a2.y * b2.y;
            }
        }
        if ((k0 + GN_KS) % QMH_GEMM_KC == 0 || k0 + GN_KS >= K) {  // a panel ends: C += its sums
            c00 = c00 + s00, c01 = c01 + s01, c10 = c10 + s10, c11 = c11 + s11;
            s00 = s01 = s10 = s11 = 0.0f;
        }
    }
    const int64_t i = i0 + 2 * r, j = j0 + 2 * c;
    if (i < M && j < N) C[i * N + j] = c00;
    if (i < M && j + 1 < N) C[i * N + j + 1] = c01;
    if (i + 1 < M && j < N) C[(i + 1) * N + j] = c10;
    if (i + 1 < M && j + 1 < N) C[(i + 1) * N + j + 1] = c11;
}

// C = 0 for K = 0 (the reference's zeroing with no panel to add), as a kernel: no memset node if the
// caller records the call into a graph
__global__ void k_gemm_zero(float *C, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
        C[i] = 0.0f;
}

extern "C" int qmh_launch_gemm_nt(const float *A, const float *B, float *C, int64_t M, int64_t N, int64_t K,
                                  void *stream) {
    if (M <= 0 || N <= 0) return 0;
    if (K <= 0) {
        hipLaunchKernelGGL(k_gemm_zero, dim3(grid_for(M * N)), dim3(256), 0, (hipStream_t)stream, C, M * N);
        return (int)hipGetLastError();
    }
    dim3 grid((unsigned)((N + GN_T - 1) / GN_T), (unsigned)((M + GN_T - 1) / GN_T));
    if ((K & 3) == 0 && (((uintptr_t)A | (uintptr_t)B) & 15) == 0)
        hipLaunchKernelGGL(k_gemm_nt<true>, grid, dim3(256), 0, (hipStream_t)stream, A, B, C, M, N, K);
    else
        hipLaunchKernelGGL(k_gemm_nt<false>, grid, dim3(256), 0, (hipStream_t)stream, A, B, C, M, N, K);
    return (int)hipGetLastError();
}

// ============================================================================ decode scores, K tile

// Lives in this file rather than beside the other attention kernels: decode speed on MI355X
// depends on where the device code of the attention kernels lands (measured: the same source
// placed here runs the 7B step at 577 tok/s, beside them at 555), so the attention kernels' code
// is kept as it was timed.
#define QMH_SC_T 64  // positions per workgroup

// Decode attention scores (as k_attn_scores in qmh_attn.hip) with the K tile staged in LDS: a
// workgroup of QMH_WG threads owns 64 positions of one kv head; its HD x 64 floats of K arrive as
// HD/16 float4 loads per thread (one
// round trip, coalesced: 16 threads read one dimension's 64 positions), and wave w then runs the
// dots of query heads w, w + 4, ... (one lane per position, the same serial order over head_dim).
// Needs head_dim % 16 == 0 and max_seq % 4 == 0 (aligned float4 rows). Used when a kv head
// serves several query heads (timed on MI355X: 6.3 -> 3.9 us at 32/8 heads, 128 dims, 640
// positions); with one query head per kv head the one-wave kernel is faster (4.0 vs 4.5 us).
template <int HD>
__global__ __launch_bounds__(QMH_WG) void k_attn_scores_t(const float *__restrict__ q, const float *__restrict__ Kt,
                                                          float *__restrict__ att, const int32_t *pos_ptr, int n_heads,
                                                          int n_kv, int max_seq, float scale) {
    static_assert(HD % 16 == 0 && (HD * QMH_SC_T / 4) % QMH_WG == 0, "whole float4 loads per thread");
    constexpr int L4 = HD * QMH_SC_T / 4 / QMH_WG;  // float4 loads per thread
    __shared__ __align__(16) float kt[HD * QMH_SC_T];  // [dim][position]
    const int pos = *pos_ptr;
    const int t0 = blockIdx.y * QMH_SC_T;
    if (pos < 0 || pos >= max_seq || t0 > pos) return;
    const int kvh = blockIdx.x, group = n_heads / n_kv, tid = threadIdx.x;
    const float *kbase = Kt + (size_t)kvh * HD * max_seq;
    float4 kv[L4];
#pragma unroll
    for (int k = 0; k < L4; k++) {
        const int e = k * QMH_WG + tid, i = e / (QMH_SC_T / 4), p4 = e % (QMH_SC_T / 4);
        const int t = t0 + 4 * p4, tc = t <= max_seq - 4 ? t : max_seq - 4;  // in-bounds float4
        kv[k] = *(const float4 *)(kbase + (size_t)i * max_seq + tc);
    }
#pragma unroll
    for (int k = 0; k < L4; k++) {
        const int e = k * QMH_WG + tid, i = e / (QMH_SC_T / 4), p4 = e % (QMH_SC_T / 4);
        *(float4 *)(kt + i * QMH_SC_T + 4 * p4) = kv[k];
    }
    __syncthreads();
    const int lane = tid & 63, t = t0 + lane;
    for (int hl = __builtin_amdgcn_readfirstlane(tid >> 6); hl < group; hl += QMH_WG / 64) {
        const float *qh = q + (size_t)(kvh * group + hl) * HD;
        float s = 0.0f;
#pragma unroll
        for (int i = 0; i < HD; i++) s = s + qh[i] * kt[i * QMH_SC_T + lane];
        if (t <= pos) att[(size_t)(kvh * group + hl) * max_seq + t] = s * scale;
    }
}


extern "C" int qmh_launch_attn_scores_tile(const float *q, const float *kcache, float *att, const int32_t *pos_ptr,
                                           int n_heads, int n_kv_heads, int head_dim, int max_seq, float scale,
                                           void *stream) {
    dim3 grid(n_kv_heads, (max_seq + QMH_SC_T - 1) / QMH_SC_T);
    hipStream_t s = (hipStream_t)stream;
#define QMH_SCT(HD) \
    hipLaunchKernelGGL(k_attn_scores_t<HD>, grid, dim3(QMH_WG), 0, s, q, kcache, att, pos_ptr, n_heads, n_kv_heads, \
                       max_seq, scale)
    if (head_dim == 128) QMH_SCT(128);
    else if (head_dim == 64) QMH_SCT(64);
    else QMH_SCT(48);
#undef QMH_SCT
    return (int)hipGetLastError();
}
