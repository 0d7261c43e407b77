// gfx950 kernels of the quillm token loop.
//
// Rounding contract: every kernel reproduces, bit for bit, the float arithmetic of the
// reference's scalar CPU path (src/kernels_scalar.c, src/ops.c, src/model.c). Integer parts
// (block dots) may be computed in any order because they are exact; float sums keep the
// reference's order (per-row serial chains), so parallelism comes from rows, heads and
// blocks, never from re-associating a float sum. The double-precision sums of RMSNorm and
// softmax are the one exception: they are tree reductions (see rmsnorm/softmax below).
#include "qmh_device.h"
#include "qmh_launch.h"

#define QMH_Q8 2
#define QMH_Q4 3

// ============================================================================ weight tiles
//
// Device layout of a quantized weight (one allocation each for codes and scales):
//   tile t covers tile_r rows; inside a tile, block b of row r sits at slot
//   s = (t*nb + b)*tile_r + r;  codes at s*CB bytes (CB = 16 for Q4_0, 32 for Q8_0),
//   scale (the block's fp16 d) at scales[s].
// A wave reading consecutive slots therefore reads consecutive 16/32-byte code chunks
// (coalesced dwordx4 loads), and the per-block partial results land in LDS in the order
// the per-row serial chain reads them. Values are the .qlm bytes, only moved.

__global__ void k_repack(const uint8_t *__restrict__ src, int64_t src_rows, int nb, int bs, int cb,
                         uint8_t *__restrict__ codes, uint16_t *__restrict__ scales, int tile_r, int64_t row_off,
                         int half) {
    int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= src_rows * nb) return;
    int64_t row = idx / nb;
    int b = (int)(idx % nb);
    const uint8_t *blk = src + (row * nb + b) * bs;
    int64_t tile, r;
    if (half < 0) {  // rows appended at row_off
        int64_t g = row_off + row;
        tile = g / tile_r;
        r = g % tile_r;
    } else {  // two matrices interleaved per tile: first half rows, then second half rows
        int hr = tile_r / 2;
        tile = row / hr;
        r = row % hr + (int64_t)half * hr;
    }
    int64_t slot = (tile * nb + b) * tile_r + r;
    scales[slot] = (uint16_t)(blk[0] | (blk[1] << 8));
    uint8_t *dst = codes + slot * cb;
    for (int i = 0; i < cb; i++) dst[i] = blk[2 + i];
}

extern "C" int qmh_launch_repack(const uint8_t *src, int64_t src_rows, int nb, int dtype, uint8_t *codes,
                                 uint16_t *scales, int tile_r, int64_t row_off, int interleave_half, void *stream) {
    int bs = dtype == QMH_Q4 ? 18 : 34, cb = dtype == QMH_Q4 ? 16 : 32;
    int64_t total = src_rows * nb;
    if (total <= 0) return 0;
    int64_t grid = (total + 255) / 256;
    hipLaunchKernelGGL(k_repack, dim3((unsigned)grid), dim3(256), 0, (hipStream_t)stream, src, src_rows, nb, bs, cb,
                       codes, scales, tile_r, row_off, interleave_half);
    return (int)hipGetLastError();
}

// ============================================================================ activation prologue
//
// Every matvec workgroup turns the f32 activation into Q8_0 blocks in its own LDS (the
// reference quantizes x once per qm_matvec, src/ops.c:59; the result is the same wherever it
// is computed). With norm_w it first applies RMSNorm (src/ops.c:93-98), so the normalised
// vector never round-trips through memory.
//   acodes[b*32 + k]: the block's 32 codes. For Q4_0 weights they are stored split, even
//                     elements in [0,16) and odd elements in [16,32), to match the weight's
//                     low/high nibbles; asum[b] = sum of the codes.
//   ad[b]            : fp32(fp16(d)) of the block.
template <bool SPLIT>
__device__ void act_prologue(const qmh_mv_args &a, int8_t *acodes, float *ad, int *asum, double *red) {
    const int n = a.cols, nb = a.nb;
    float inv = 1.0f;
    if (a.norm_w) {
        double ss = 0.0;
        for (int i = threadIdx.x; i < n; i += blockDim.x) {
            double v = (double)a.x[i];
            ss += v * v;
        }
        ss = qmh_block_sum_d(ss, red);
        inv = (float)(1.0 / sqrt(ss / (double)n + (double)a.eps));
    }
    const int sub = threadIdx.x & 7;
    const int per_pass = blockDim.x >> 3;
    for (int b0 = 0; b0 < nb; b0 += per_pass) {
        const int b = b0 + (threadIdx.x >> 3);
        const bool on = b < nb;
        float v[4];
        float m = 0.0f;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            int i = b * 32 + sub * 4 + k;
            float xv = (on && i < n) ? a.x[i] : 0.0f;
            if (a.norm_w && on && i < n) xv = xv * inv * a.norm_w[i];
            v[k] = xv;
            float av = fabsf(xv);
            m = av > m ? av : m;
        }
        m = qmh_amax8(m);
        uint16_t dh = qmh_f2h(m / 127.0f);
        float dd = qmh_h2f(dh);
        int q[4];
#pragma unroll
        for (int k = 0; k < 4; k++) q[k] = qmh_q8_code(v[k], dd);
        int ps = q[0] + q[1] + q[2] + q[3];
        ps += __shfl_xor(ps, 1);
        ps += __shfl_xor(ps, 2);
        ps += __shfl_xor(ps, 4);
        if (on) {
            int8_t *c = acodes + b * 32;
            if (SPLIT) {
                c[sub * 2 + 0] = (int8_t)q[0];
                c[sub * 2 + 1] = (int8_t)q[2];
                c[16 + sub * 2 + 0] = (int8_t)q[1];
                c[16 + sub * 2 + 1] = (int8_t)q[3];
            } else {
#pragma unroll
                for (int k = 0; k < 4; k++) c[sub * 4 + k] = (int8_t)q[k];
            }
            if (sub == 0) {
                ad[b] = dd;
                asum[b] = ps;
            }
            if (a.xq_out && blockIdx.x == 0) {
                uint8_t *o = a.xq_out + (size_t)b * 34;
                if (sub == 0) {
                    o[0] = (uint8_t)(dh & 0xff);
                    o[1] = (uint8_t)(dh >> 8);
                }
#pragma unroll
                for (int k = 0; k < 4; k++) o[2 + sub * 4 + k] = (uint8_t)(int8_t)q[k];
            }
        }
    }
    __syncthreads();
}

// ============================================================================ epilogues

// y: the row's result; lanes of one tile hold consecutive rows, so the RoPE partner of row
// 2i/2i+1 is lane ^ 1 and the W3 partner of an interleaved W1 row is lane + 16.
__device__ __forceinline__ void mv_epilogue(const qmh_mv_args &a, int row, float y, int lane_in_tile) {
    switch (a.epi) {
    case QMH_EPI_STORE:
        if (row < a.rows) a.out0[row] = y;
        break;
    case QMH_EPI_ADD:
        if (row < a.rows) a.out0[row] = a.out0[row] + y;
        break;
    case QMH_EPI_QKV: {
        const float partner = __shfl_xor(y, 1);
        const int pos = *a.pos_ptr;
        // the position comes from device memory: never let a stale one address past the cache
        if (row >= a.rows || pos < 0 || pos >= a.max_seq) break;
        if (row < a.seg2) {  // q or k: rotate the (2i, 2i+1) pair, src/ops.c:114-126
            const int local = row < a.seg1 ? row : row - a.seg1;
            const int i = (local % a.head_dim) >> 1;
            const float *cs = a.rope + ((size_t)pos * (a.head_dim >> 1) + i) * 2;
            const float c = cs[0], s = cs[1];
            float v = (local & 1) == 0 ? (y * c - partner * s) : (partner * s + y * c);
            if (row < a.seg1) a.out0[local] = v;
            else a.out1[(size_t)pos * a.kvd + local] = v;
        } else {  // v: transposed cache [kvd][max_seq]
            a.out2[(size_t)(row - a.seg2) * a.max_seq + pos] = y;
        }
        break;
    }
    case QMH_EPI_SWIGLU: {
        const float up = __shfl_down(y, 16);  // lane j < 16 holds W1 row, lane j+16 the W3 row
        if (lane_in_tile < 16 && row < a.rows) a.out0[row] = y / (1.0f + qmh_expf(-y)) * up;
        break;
    }
    }
}

// ============================================================================ quantized matvec
//
// y = W x with W Q4_0 or Q8_0 and x quantized to Q8_0 (src/ops.c:36-61), one row's dot as in
// src/kernels_scalar.c:12-34:  s = +0; for b: s = s + (float)acc_b * (d_w,b * d_x,b).
//
// Workgroup = 256 threads, grid-stride over tiles of R rows. Per tile:
//   1. every thread owns blocks l = chunk*256*CH + k*256 + tid of the tile (coalesced code and
//      scale loads; the next chunk's loads are issued before this chunk is computed),
//   2. computes the exact int32 block dot against the LDS activation and the block term
//      t = (float)acc * (d_w*d_x), written to T[l] in LDS,
//   3. lanes 0..R-1 of wave 0 run each row's serial chain over its nb terms (the reference's
//      summation order), then the epilogue.
template <int WT, int R>
__global__ __launch_bounds__(QMH_WG) void k_matvec(qmh_mv_args a) {
    constexpr int CB = WT == QMH_Q4 ? 16 : 32;  // code bytes per block
    constexpr int NV = CB / 16;                 // uint4 per block
    constexpr int CH = WT == QMH_Q4 ? 8 : 4;    // blocks per thread per chunk
    constexpr int CHUNK = QMH_WG * CH;
    extern __shared__ __align__(16) uint8_t smem[];
    __shared__ double red[16];

    const int nb = a.nb, TB = R * nb, nchunk = (TB + CHUNK - 1) / CHUNK;
    const int tid = threadIdx.x;
    int tile = blockIdx.x;
    if (tile >= a.ntiles) return;

    int8_t *acodes = (int8_t *)smem;
    float *ad = (float *)(smem + (size_t)nb * 32);
    int *asum = (int *)(smem + (size_t)nb * 36);
    float *T = (float *)(smem + (size_t)nb * 40);

    const uint4 *codes = (const uint4 *)a.codes;
    uint4 A[CH][NV], B[CH][NV];
    uint16_t As[CH], Bs[CH];

#define QMH_LOAD(BUF, BS, TILE, CHK)                                                   \
    {                                                                                  \
        const size_t tbase = (size_t)(TILE) * TB;                                      \
        _Pragma("unroll") for (int k = 0; k < CH; k++) {                               \
            const int l = (CHK) * CHUNK + k * QMH_WG + tid;                            \
            if (l < TB) {                                                              \
                const size_t slot = tbase + l;                                         \
                _Pragma("unroll") for (int v = 0; v < NV; v++) BUF[k][v] = codes[slot * NV + v]; \
                BS[k] = a.scales[slot];                                                \
            }                                                                          \
        }                                                                              \
    }

    QMH_LOAD(A, As, tile, 0);
    act_prologue<WT == QMH_Q4>(a, acodes, ad, asum, red);

    int c = 0;
    for (;;) {
        int nt = tile, nc = c + 1;
        if (nc == nchunk) {
            nt = tile + gridDim.x;
            nc = 0;
        }
        const bool more = nt < a.ntiles;
        if (more) QMH_LOAD(B, Bs, nt, nc);
#pragma unroll
        for (int k = 0; k < CH; k++) {
            const int l = c * CHUNK + k * QMH_WG + tid;
            if (l < TB) {
                const int b = l / R;
                const int4 *xv = (const int4 *)(acodes + b * 32);
                const int4 x0 = xv[0], x1 = xv[1];
                int acc;
                if (WT == QMH_Q4) {
                    const uint4 w = A[k][0];
                    acc = 0;
                    acc = __builtin_amdgcn_sdot4((int)(w.x & 0x0f0f0f0fu), x0.x, acc, false);
                    acc = __builtin_amdgcn_sdot4((int)((w.x >> 4) & 0x0f0f0f0fu), x1.x, acc, false);
                    acc = __builtin_amdgcn_sdot4((int)(w.y & 0x0f0f0f0fu), x0.y, acc, false);
                    acc = __builtin_amdgcn_sdot4((int)((w.y >> 4) & 0x0f0f0f0fu), x1.y, acc, false);
                    acc = __builtin_amdgcn_sdot4((int)(w.z & 0x0f0f0f0fu), x0.z, acc, false);
                    acc = __builtin_amdgcn_sdot4((int)((w.z >> 4) & 0x0f0f0f0fu), x1.z, acc, false);
                    acc = __builtin_amdgcn_sdot4((int)(w.w & 0x0f0f0f0fu), x0.w, acc, false);
                    acc = __builtin_amdgcn_sdot4((int)((w.w >> 4) & 0x0f0f0f0fu), x1.w, acc, false);
                    acc -= 8 * asum[b];  // sum (q-8)*x = sum q*x - 8*sum x, exact
                } else {
                    const uint4 w0 = A[k][0], w1 = A[k][NV - 1];
                    acc = 0;
                    acc = __builtin_amdgcn_sdot4((int)w0.x, x0.x, acc, false);
                    acc = __builtin_amdgcn_sdot4((int)w0.y, x0.y, acc, false);
                    acc = __builtin_amdgcn_sdot4((int)w0.z, x0.z, acc, false);
                    acc = __builtin_amdgcn_sdot4((int)w0.w, x0.w, acc, false);
                    acc = __builtin_amdgcn_sdot4((int)w1.x, x1.x, acc, false);
                    acc = __builtin_amdgcn_sdot4((int)w1.y, x1.y, acc, false);
                    acc = __builtin_amdgcn_sdot4((int)w1.z, x1.z, acc, false);
                    acc = __builtin_amdgcn_sdot4((int)w1.w, x1.w, acc, false);
                }
                T[l] = (float)acc * (qmh_h2f(As[k]) * ad[b]);
            }
        }
        if (c == nchunk - 1) {
            __syncthreads();
            if (tid < R) {
                float s = 0.0f;
                for (int b = 0; b < nb; b++) s = s + T[b * R + tid];
                const int row = R == QMH_TILE_R ? tile * R + tid : tile * (R / 2) + (tid & (R / 2 - 1));
                mv_epilogue(a, row, s, tid);
            }
            __syncthreads();
        }
        if (!more) break;
#pragma unroll
        for (int k = 0; k < CH; k++) {
            As[k] = Bs[k];
#pragma unroll
            for (int v = 0; v < NV; v++) A[k][v] = B[k][v];
        }
        tile = nt;
        c = nc;
    }
#undef QMH_LOAD
}

// f32 weights (src/kernels_scalar.c:6-10 via src/ops.c:42-45): lane per row, x in LDS,
// s = +0; s = s + w_i*x_i in index order.
__global__ __launch_bounds__(QMH_WG) void k_matvec_f32(qmh_mv_args a) {
    extern __shared__ __align__(16) uint8_t smem[];
    __shared__ double red[16];
    float *xs = (float *)smem;
    const int n = a.cols;
    float inv = 1.0f;
    if (a.norm_w) {
        double ss = 0.0;
        for (int i = threadIdx.x; i < n; i += blockDim.x) {
            double v = (double)a.x[i];
            ss += v * v;
        }
        ss = qmh_block_sum_d(ss, red);
        inv = (float)(1.0 / sqrt(ss / (double)n + (double)a.eps));
    }
    for (int i = threadIdx.x; i < n; i += blockDim.x) xs[i] = a.norm_w ? a.x[i] * inv * a.norm_w[i] : a.x[i];
    __syncthreads();
    const int row = blockIdx.x * blockDim.x + threadIdx.x;
    const float *w = (const float *)a.codes + (size_t)(row < a.rows ? row : 0) * n;
    float s = 0.0f;
    for (int i = 0; i < n; i++) s = s + w[i] * xs[i];
    mv_epilogue(a, row, s, threadIdx.x & 15);
}

extern "C" int qmh_launch_matvec(const qmh_mv_args *a, int grid_cap, void *stream) {
    const int grid = a->ntiles < grid_cap ? a->ntiles : grid_cap;
    const size_t lds = (size_t)a->nb * 40 + (size_t)a->tile_r * a->nb * 4;
    hipStream_t s = (hipStream_t)stream;
    if (a->dtype == QMH_Q4 && a->tile_r == 16) hipLaunchKernelGGL((k_matvec<QMH_Q4, 16>), dim3(grid), dim3(QMH_WG), lds, s, *a);
    else if (a->dtype == QMH_Q4 && a->tile_r == 32) hipLaunchKernelGGL((k_matvec<QMH_Q4, 32>), dim3(grid), dim3(QMH_WG), lds, s, *a);
    else if (a->dtype == QMH_Q8 && a->tile_r == 16) hipLaunchKernelGGL((k_matvec<QMH_Q8, 16>), dim3(grid), dim3(QMH_WG), lds, s, *a);
    else if (a->dtype == QMH_Q8 && a->tile_r == 32) hipLaunchKernelGGL((k_matvec<QMH_Q8, 32>), dim3(grid), dim3(QMH_WG), lds, s, *a);
    else return (int)hipErrorInvalidValue;
    return (int)hipGetLastError();
}

extern "C" int qmh_launch_matvec_f32(const qmh_mv_args *a, void *stream) {
    const int grid = (a->rows + QMH_WG - 1) / QMH_WG;
    hipLaunchKernelGGL(k_matvec_f32, dim3(grid), dim3(QMH_WG), (size_t)a->cols * 4, (hipStream_t)stream, *a);
    return (int)hipGetLastError();
}

// ============================================================================ embedding

// x = dequantised row `token` of tok_embd (src/model.c:162 -> src/quant.c:65-101)
__global__ void k_embed(const uint8_t *__restrict__ E, int dtype, int dim, int vocab, const int32_t *tok_ptr,
                        float *x) {
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
                                float *x, void *stream) {
    hipLaunchKernelGGL(k_embed, dim3((dim + 255) / 256), dim3(256), 0, (hipStream_t)stream, tok_embd, dtype, dim,
                       vocab, tok_ptr, x);
    return (int)hipGetLastError();
}

// ============================================================================ attention
//
// Reference src/model.c:127-156, per head h (kv head h/group):
//   att[t] = dot_f32(q_h, K[t]) * scale      serial fp32 dot over head_dim
//   softmax(att[0..pos])                     max, expf, double sum, * (float)(1/sum)
//   out[i] = +0; out[i] = out[i] + att[t]*V[t][i] for t = 0..pos in order
// K cache: [max_seq][kvd] per layer (as the reference). V cache is stored transposed,
// [kvd][max_seq], so the serial chain over t for one output column reads contiguous memory.

#define QMH_ATT_TT 64  // positions per scores workgroup

__global__ __launch_bounds__(QMH_WG) void k_attn_scores(const float *__restrict__ q, const float *__restrict__ K,
                                                        float *__restrict__ att, const int32_t *pos_ptr, int n_heads,
                                                        int n_kv, int hd, int max_seq, float scale) {
    extern __shared__ __align__(16) uint8_t smem[];
    const int pos = *pos_ptr;
    const int t0 = blockIdx.y * QMH_ATT_TT;
    if (pos < 0 || pos >= max_seq || t0 > pos) return;
    const int nt = min(QMH_ATT_TT, pos + 1 - t0);
    const int kvh = blockIdx.x, group = n_heads / n_kv, kvd = hd * n_kv;
    float *Ks = (float *)smem;                       // [QMH_ATT_TT][hd+1]
    float *Qs = Ks + QMH_ATT_TT * (hd + 1);          // [group][hd]
    for (int e = threadIdx.x; e < nt * hd; e += blockDim.x) {
        const int t = e / hd, i = e % hd;
        Ks[t * (hd + 1) + i] = K[(size_t)(t0 + t) * kvd + kvh * hd + i];
    }
    for (int e = threadIdx.x; e < group * hd; e += blockDim.x) Qs[e] = q[(size_t)kvh * group * hd + e];
    __syncthreads();
    for (int p = threadIdx.x; p < group * nt; p += blockDim.x) {
        const int hl = p / nt, t = p % nt;
        const float *qh = Qs + hl * hd, *kt = Ks + t * (hd + 1);
        float s = 0.0f;
        for (int i = 0; i < hd; i++) s = s + qh[i] * kt[i];
        att[(size_t)(kvh * group + hl) * max_seq + t0 + t] = s * scale;
    }
}

#define QMH_PV_CW 16   // output columns per workgroup
#define QMH_PV_TC 512  // positions per LDS chunk

__global__ __launch_bounds__(QMH_WG) void k_attn_pv(const float *__restrict__ att, const float *__restrict__ Vt,
                                                    float *__restrict__ out, const int32_t *pos_ptr, int n_heads,
                                                    int n_kv, int hd, int max_seq) {
    extern __shared__ __align__(16) uint8_t smem[];
    __shared__ double red[16];
    __shared__ float redf[16];
    __shared__ float mx_s[16], inv_s[16];
    const int n = *pos_ptr + 1;
    if (n < 1 || n > max_seq) return;  // stale position in device memory: touch nothing
    const int kvh = blockIdx.x, i0 = blockIdx.y * QMH_PV_CW, group = n_heads / n_kv;
    float *P = (float *)smem;                      // [group][TC]
    float *Vs = P + group * QMH_PV_TC;             // [CW][TC+1]
    // softmax statistics per head of the group (src/ops.c:100-112)
    for (int hl = 0; hl < group; hl++) {
        const float *s = att + (size_t)(kvh * group + hl) * max_seq;
        float m = -__builtin_inff();
        for (int t = threadIdx.x; t < n; t += blockDim.x) m = s[t] > m ? s[t] : m;
        m = qmh_block_max(m, redf);
        double sum = 0.0;
        for (int t = threadIdx.x; t < n; t += blockDim.x) sum += (double)qmh_expf(s[t] - m);
        sum = qmh_block_sum_d(sum, red);
        if (threadIdx.x == 0) {
            mx_s[hl] = m;
            inv_s[hl] = (float)(1.0 / sum);
        }
    }
    __syncthreads();
    const int lane_h = threadIdx.x / QMH_PV_CW, col = threadIdx.x % QMH_PV_CW;
    const bool chain = lane_h < group;
    float acc = 0.0f;
    for (int t0 = 0; t0 < n; t0 += QMH_PV_TC) {
        const int nt = min(QMH_PV_TC, n - t0);
        for (int e = threadIdx.x; e < group * nt; e += blockDim.x) {
            const int hl = e / nt, t = e % nt;
            const float sv = att[(size_t)(kvh * group + hl) * max_seq + t0 + t];
            P[hl * QMH_PV_TC + t] = qmh_expf(sv - mx_s[hl]) * inv_s[hl];
        }
        for (int e = threadIdx.x; e < QMH_PV_CW * nt; e += blockDim.x) {
            const int cc = e / nt, t = e % nt;
            const int i = i0 + cc;
            Vs[cc * (QMH_PV_TC + 1) + t] = i < hd ? Vt[(size_t)(kvh * hd + i) * max_seq + t0 + t] : 0.0f;
        }
        __syncthreads();
        if (chain) {
            const float *p = P + lane_h * QMH_PV_TC, *v = Vs + col * (QMH_PV_TC + 1);
            for (int t = 0; t < nt; t++) acc = acc + p[t] * v[t];
        }
        __syncthreads();
    }
    if (chain && i0 + col < hd) out[(size_t)(kvh * group + lane_h) * hd + i0 + col] = acc;
}

extern "C" int qmh_launch_attn_scores(const float *q, const float *kcache, float *att, const int32_t *pos_ptr,
                                      int n_heads, int n_kv_heads, int head_dim, int max_seq, float scale, void *stream) {
    const int group = n_heads / n_kv_heads;
    const size_t lds = ((size_t)QMH_ATT_TT * (head_dim + 1) + (size_t)group * head_dim) * 4;
    dim3 grid(n_kv_heads, (max_seq + QMH_ATT_TT - 1) / QMH_ATT_TT);
    hipLaunchKernelGGL(k_attn_scores, grid, dim3(QMH_WG), lds, (hipStream_t)stream, q, kcache, att, pos_ptr, n_heads,
                       n_kv_heads, head_dim, max_seq, scale);
    return (int)hipGetLastError();
}

extern "C" int qmh_launch_attn_pv(const float *att, const float *vtcache, float *out, const int32_t *pos_ptr,
                                  int n_heads, int n_kv_heads, int head_dim, int max_seq, void *stream) {
    const int group = n_heads / n_kv_heads;
    if (group > 16 || group * QMH_PV_CW > QMH_WG) return (int)hipErrorInvalidValue;
    const size_t lds = ((size_t)group * QMH_PV_TC + (size_t)QMH_PV_CW * (QMH_PV_TC + 1)) * 4;
    dim3 grid(n_kv_heads, (head_dim + QMH_PV_CW - 1) / QMH_PV_CW);
    hipLaunchKernelGGL(k_attn_pv, grid, dim3(QMH_WG), lds, (hipStream_t)stream, att, vtcache, out, pos_ptr, n_heads,
                       n_kv_heads, head_dim, max_seq);
    return (int)hipGetLastError();
}

// ============================================================================ argmax

// first index of the maximum (src/sampler.c:27-32): each thread keeps the first strict
// maximum of its stride, and pairs combine preferring the larger value, then the lower index.
__global__ __launch_bounds__(1024) void k_argmax(const float *__restrict__ x, int n, int32_t *out_idx,
                                                 int32_t *tokpos, int32_t *record, int record_cap) {
    __shared__ float bv[16];
    __shared__ int bi[16];
    float v = -__builtin_inff();
    int idx = 0x7fffffff;
    for (int i = threadIdx.x; i < n; i += blockDim.x)
        if (idx == 0x7fffffff || x[i] > v) {
            v = x[i];
            idx = i;
        }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        float ov = __shfl_xor(v, o);
        int oi = __shfl_xor(idx, o);
        if (ov > v || (ov == v && oi < idx)) {
            v = ov;
            idx = oi;
        }
    }
    const int w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) {
        bv[w] = v;
        bi[w] = idx;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        const int nw = blockDim.x >> 6;
        for (int k = 1; k < nw; k++)
            if (bv[k] > v || (bv[k] == v && bi[k] < idx)) {
                v = bv[k];
                idx = bi[k];
            }
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
    hipLaunchKernelGGL(k_argmax, dim3(1), dim3(1024), 0, (hipStream_t)stream, x, n, out_idx, tokpos, record,
                       record_cap);
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
    const float qmax = dtype == QMH_Q4 ? 7.0f : 127.0f;
    const uint16_t dh = qmh_f2h(m / qmax);
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
#pragma unroll
        for (int k = 0; k < 4; k++) o[2 + sub * 4 + k] = (uint8_t)(int8_t)qmh_q8_code(v[k], dd);
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

// RMSNorm (src/ops.c:93-98): one workgroup; double sum of squares as a fixed tree, then
// out = (x*inv)*w. The tree sum can differ from the reference's serial double sum in its
// last bits; the fp32 inv it rounds to is the same unless the two straddle a rounding point.
__global__ __launch_bounds__(1024) void k_rmsnorm(float *out, const float *x, const float *w, int64_t n, float eps) {
    __shared__ double red[16];
    double ss = 0.0;
    for (int64_t i = threadIdx.x; i < n; i += blockDim.x) ss += (double)x[i] * (double)x[i];
    ss = qmh_block_sum_d(ss, red);
    const float inv = (float)(1.0 / sqrt(ss / (double)n + (double)eps));
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
    const float inv = (float)(1.0 / sum);
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
// panels of 256 (QM_GEMM_KC, src/kernels.h:37); each panel is a serial fp32 sum from +0 and
// the panel sums are added to C (from +0) in order. 16x16 outputs per workgroup, panels of A
// and B staged in LDS (padded rows: conflict-free column walks).
#define QMH_GEMM_KC 256
__global__ __launch_bounds__(256) void k_gemm_nt(const float *__restrict__ A, const float *__restrict__ B,
                                                 float *__restrict__ C, int64_t M, int64_t N, int64_t K) {
    __shared__ float As[16][QMH_GEMM_KC + 1], Bs[16][QMH_GEMM_KC + 1];
    const int ty = threadIdx.x / 16, tx = threadIdx.x % 16;
    const int64_t i = (int64_t)blockIdx.y * 16 + ty, j = (int64_t)blockIdx.x * 16 + tx;
    float c = 0.0f;
    for (int64_t k0 = 0; k0 < K; k0 += QMH_GEMM_KC) {
        const int kc = (int)(K - k0 < QMH_GEMM_KC ? K - k0 : QMH_GEMM_KC);
        for (int e = threadIdx.x; e < 16 * kc; e += 256) {
            const int r = e / kc, k = e % kc;
            const int64_t ai = (int64_t)blockIdx.y * 16 + r, bj = (int64_t)blockIdx.x * 16 + r;
            As[r][k] = ai < M ? A[ai * K + k0 + k] : 0.0f;
            Bs[r][k] = bj < N ? B[bj * K + k0 + k] : 0.0f;
        }
        __syncthreads();
        float acc = 0.0f;
        for (int k = 0; k < kc; k++) acc = acc + As[ty][k] * Bs[tx][k];
        c = c + acc;
        __syncthreads();
    }
    if (i < M && j < N) C[i * N + j] = c;
}

extern "C" int qmh_launch_gemm_nt(const float *A, const float *B, float *C, int64_t M, int64_t N, int64_t K,
                                  void *stream) {
    if (M <= 0 || N <= 0) return 0;
    dim3 grid((unsigned)((N + 15) / 16), (unsigned)((M + 15) / 16));
    hipLaunchKernelGGL(k_gemm_nt, grid, dim3(256), 0, (hipStream_t)stream, A, B, C, M, N, K);
    return (int)hipGetLastError();
}
