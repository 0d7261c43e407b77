// gfx950 matrix-vector kernels of the quillm token loop (Q4_0 / Q8_0 / f32 weights).
//
// Rounding contract: results are bit-identical to the reference's scalar CPU path. The
// int32 block dots are exact in any order; every float sum keeps the reference's order
// (one serial chain per row), so parallelism comes from rows and blocks, never from
// re-associating a float sum. Built with -ffp-contract=off (no a*b+c fusion).
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
// A wave reading consecutive slots reads consecutive 16/32-byte code chunks (coalesced
// dwordx4 loads). Values are the .qlm bytes, only moved.

__global__ void k_repack(const uint8_t *__restrict__ src, int64_t src_rows, int nb, int bs, int cb,
                         uint8_t *__restrict__ codes, uint16_t *__restrict__ scales, int tile_r, int64_t row_off,
                         int half, int64_t nslots) {
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
    if (slot >= nslots) return;  // the host sized the tiles wrongly: write nothing out of bounds
    scales[slot] = (uint16_t)(blk[0] | (blk[1] << 8));
    uint8_t *dst = codes + slot * cb;
    for (int i = 0; i < cb; i++) dst[i] = blk[2 + i];
}

extern "C" int qmh_launch_repack(const uint8_t *src, int64_t src_rows, int nb, int dtype, uint8_t *codes,
                                 uint16_t *scales, int tile_r, int64_t row_off, int interleave_half, int64_t nslots,
                                 void *stream) {
    int bs = dtype == QMH_Q4 ? 18 : 34, cb = dtype == QMH_Q4 ? 16 : 32;
    int64_t total = src_rows * nb;
    if (total <= 0) return 0;
    int64_t grid = (total + 255) / 256;
    hipLaunchKernelGGL(k_repack, dim3((unsigned)grid), dim3(256), 0, (hipStream_t)stream, src, src_rows, nb, bs, cb,
                       codes, scales, tile_r, row_off, interleave_half, nslots);
    return (int)hipGetLastError();
}

// ============================================================================ activation
//
// Every matvec workgroup turns the f32 activation into Q8_0 blocks in its own LDS (the
// reference quantizes x once per qm_matvec, src/ops.c:59; the result is the same wherever it
// is computed). With RMSNorm (NORM) the gain is applied first (src/ops.c:93-98), so the
// normalised vector never round-trips through memory.
//
// Thread t holds 8 consecutive elements (two float4) of x (and of the gain) for every pass k:
// elements 8*(k*NT + t) .. +7, i.e. a quarter of block k*NT/4 + t/4. The loads are coalesced and
// issued BEFORE the weight loads (the vector-memory counter retires loads in order, so the
// prologue never waits for weights); the 4 lanes of a block reduce its amax and code sum with
// two DPP steps. Results in LDS, one 48-byte record per block:
//   codes[b*48 + k]: the block's 32 codes. For Q4_0 weights they are stored split, even
//                    elements in [0,16) and odd elements in [16,32), to match the weight's
//                    low/high nibbles;
//   d[b*12]        : fp32(fp16(d)) of the block;  sum[b*12]: the sum of its codes.

// float4 pairs of the activation per thread (passes) for NT threads: cols <= P*8*NT, at least
// 6144 with RMSNorm and 12288 without
template <bool NORM, int NT>
struct ActRegs {
    static constexpr int P = ((NORM ? 6144 : 12288) + 8 * NT - 1) / (8 * NT);
};

// x (and gain) float4 pairs of the passes that hold blocks; lanes past the end read the last
// whole float4 (the values are masked later). A row length that is not a multiple of 4 takes
// scalar loads.
template <bool NORM, int NT>
__device__ __forceinline__ void act_load(const qmh_mv_args &a, float4 *xr, float4 *wr) {
    constexpr int P = ActRegs<NORM, NT>::P;
    const int n = a.cols, tid = threadIdx.x;
    if ((n & 3) == 0) {
        const int q_last = (n >> 2) - 1;
        const float4 *x4 = (const float4 *)a.x, *w4 = (const float4 *)a.norm_w;
#pragma unroll
        for (int k = 0; k < P; k++)
            if (k * NT * 8 < n) {
#pragma unroll
                for (int h = 0; h < 2; h++) {
                    const int q = 2 * (k * NT + tid) + h, qc = q < q_last ? q : q_last;
                    xr[2 * k + h] = x4[qc];
                    if (NORM) wr[2 * k + h] = w4[qc];
                }
            }
    } else {
#pragma unroll
        for (int k = 0; k < P; k++)
            if (k * NT * 8 < n) {
#pragma unroll
                for (int h = 0; h < 2; h++) {
                    float xv[4], wv[4];
#pragma unroll
                    for (int j = 0; j < 4; j++) {
                        const int i = 8 * (k * NT + tid) + 4 * h + j, ic = i < n ? i : n - 1;
                        xv[j] = a.x[ic];
                        wv[j] = NORM ? a.norm_w[ic] : 0.0f;
                    }
                    xr[2 * k + h] = make_float4(xv[0], xv[1], xv[2], xv[3]);
                    if (NORM) wr[2 * k + h] = make_float4(wv[0], wv[1], wv[2], wv[3]);
                }
            }
    }
}

// Where the quantized blocks go in LDS: block b's codes at codes + r*cs, its d and code sum at
// d[r*ds], sum[r*ds], for every record r = b, b + nb, b + 2nb, ... below nrec.
struct ActDst {
    int8_t *codes;
    int cs;
    float *d;
    int *sum;
    int ds, nrec;
};

template <bool SPLIT, bool NORM, int NT>
__device__ void act_finish(const qmh_mv_args &a, const float4 *xr, const float4 *wr, const ActDst &dst,
                           double *red) {
    constexpr int P = ActRegs<NORM, NT>::P;
    const int n = a.cols, nb = a.nb, tid = threadIdx.x, sub = tid & 3;
    float inv = 1.0f;
    if (NORM) {
        double ss = 0.0;
#pragma unroll
        for (int k = 0; k < P; k++)
            if (k * NT * 8 < n) {
                const float xa[8] = {xr[2 * k].x,     xr[2 * k].y,     xr[2 * k].z,     xr[2 * k].w,
                                     xr[2 * k + 1].x, xr[2 * k + 1].y, xr[2 * k + 1].z, xr[2 * k + 1].w};
#pragma unroll
                for (int j = 0; j < 8; j++) {
                    const float xv = 8 * (k * NT + tid) + j < n ? xa[j] : 0.0f;
                    ss += (double)xv * (double)xv;
                }
            }
        // workgroup sum: wave butterflies, then the waves in order (red is not reused, so one
        // barrier publishes the partials)
        ss = qmh_wave_sum_d(ss);
        if ((tid & 63) == 0) red[tid >> 6] = ss;
        __syncthreads();
        ss = 0.0;
#pragma unroll
        for (int w = 0; w < NT / 64; w++) ss += red[w];
        // same ss in every thread: uniform branches
        // (a.exact_norm, tests: always the serial sum)
        if (a.exact_norm || !qmh_rms_inv_margin(ss, n, nb * 32, a.eps, &inv)) {
            const double d = qmh_sum_slack(ss, nb * 32);
            inv = qmh_rms_inv(ss - d, n, a.eps);
            if (a.exact_norm || inv != qmh_rms_inv(ss + d, n, a.eps)) {
                if (tid == 0) {
                    double s = 0.0;
                    for (int i = 0; i < n; i++) s += (double)a.x[i] * (double)a.x[i];
                    red[15] = s;  // red[0 .. NT/64) hold the partials; 15 is free
                }
                __syncthreads();
                inv = qmh_rms_inv(red[15], n, a.eps);
            }
        }
    }
#pragma unroll
    for (int k = 0; k < P; k++) {
        if (k * (NT / 4) >= nb) break;  // uniform
        const int b = k * (NT / 4) + (tid >> 2), i8 = 8 * (k * NT + tid);
        const bool on = b < nb;
        const float xa[8] = {xr[2 * k].x,     xr[2 * k].y,     xr[2 * k].z,     xr[2 * k].w,
                             xr[2 * k + 1].x, xr[2 * k + 1].y, xr[2 * k + 1].z, xr[2 * k + 1].w};
        float wa[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
        if (NORM) {
            wa[0] = wr[2 * k].x;
            wa[1] = wr[2 * k].y;
            wa[2] = wr[2 * k].z;
            wa[3] = wr[2 * k].w;
            wa[4] = wr[2 * k + 1].x;
            wa[5] = wr[2 * k + 1].y;
            wa[6] = wr[2 * k + 1].z;
            wa[7] = wr[2 * k + 1].w;
        }
        float v[8], m = 0.0f;
#pragma unroll
        for (int j = 0; j < 8; j++) {
            float xv = (on && i8 + j < n) ? xa[j] : 0.0f;
            if (NORM) xv = xv * inv * wa[j];  // (x*inv)*w as the reference; 0 stays 0 past n
            v[j] = xv;
            const float av = fabsf(xv);
            m = av > m ? av : m;
        }
        m = qmh_amax4(m);
        const uint16_t dh = qmh_f2h(qmh_div127(m));
        const float dd = qmh_h2f(dh), rinv = qmh_rcp(dd);
        int q[8];
        qmh_q8_codes4(v, dd, rinv, q);
        qmh_q8_codes4(v + 4, dd, rinv, q + 4);
        const int ps = qmh_sum4(q[0] + q[1] + q[2] + q[3] + q[4] + q[5] + q[6] + q[7]);
        if (on) {
            uint2 w;  // the lane's 8 codes: SPLIT, evens then odds; else in order
            if (SPLIT) {
                w.x = (uint32_t)((q[0] & 0xff) | ((q[2] & 0xff) << 8) | ((q[4] & 0xff) << 16) | ((uint32_t)(q[6] & 0xff) << 24));
                w.y = (uint32_t)((q[1] & 0xff) | ((q[3] & 0xff) << 8) | ((q[5] & 0xff) << 16) | ((uint32_t)(q[7] & 0xff) << 24));
            } else {
                w.x = (uint32_t)((q[0] & 0xff) | ((q[1] & 0xff) << 8) | ((q[2] & 0xff) << 16) | ((uint32_t)(q[3] & 0xff) << 24));
                w.y = (uint32_t)((q[4] & 0xff) | ((q[5] & 0xff) << 8) | ((q[6] & 0xff) << 16) | ((uint32_t)(q[7] & 0xff) << 24));
            }
            for (int rb = b; rb < dst.nrec; rb += nb) {
                int8_t *c = dst.codes + rb * dst.cs;
                if (SPLIT) {
                    *(uint32_t *)(c + sub * 4) = w.x;
                    *(uint32_t *)(c + 16 + sub * 4) = w.y;
                } else {
                    *(uint2 *)(c + sub * 8) = w;
                }
                if (sub == 0) {
                    dst.d[rb * dst.ds] = dd;
                    dst.sum[rb * dst.ds] = ps;
                }
            }
            if (a.xq_out && blockIdx.x == 0) {
                uint8_t *o = a.xq_out + (size_t)b * 34;
                if (sub == 0) {
                    o[0] = (uint8_t)(dh & 0xff);
                    o[1] = (uint8_t)(dh >> 8);
                }
#pragma unroll
                for (int j = 0; j < 8; j++) o[2 + sub * 8 + j] = (uint8_t)(int8_t)q[j];
            }
        }
    }
    __syncthreads();
}

// ============================================================================ epilogue

// Values an epilogue reads from memory, fetched before the next chunk's weight loads.
struct EpiIn {
    float resid;  // EPI_ADD: the residual x[row]
    float c, s;   // EPI_QKV: RoPE factors of the row's pair at pos
};

__device__ __forceinline__ EpiIn epi_fetch(const qmh_mv_args &a, int row, int pos) {
    EpiIn e = {0.0f, 1.0f, 0.0f};
    const int rc = row < a.rows ? row : a.rows - 1;
    if (a.epi == QMH_EPI_ADD) e.resid = a.out0[rc];
    if (a.epi == QMH_EPI_QKV) {
        const int local = rc < a.seg1 ? rc : (rc < a.seg2 ? rc - a.seg1 : 0);
        const int i = (local % a.head_dim) >> 1;
        const int p = pos < 0 ? 0 : (pos >= a.max_seq ? a.max_seq - 1 : pos);
        const float2 cs = *(const float2 *)(a.rope + ((size_t)p * (a.head_dim >> 1) + i) * 2);
        e.c = cs.x;
        e.s = cs.y;
    }
    return e;
}

// Max and sum over lanes 0..31 of a wave, every lane ending with the result: DPP inside groups
// of 8, then lane ^ 8 (row rotate by 8), then lanes 0 and 16 read as scalars. The max takes
// non-negative values with no NaN.
#define MV_DPP_ROW_ROR8 0x128
__device__ __forceinline__ float mv_amax32(float m) {
    m = qmh_amax8(m);
    const float p = __int_as_float(qmh_dpp<MV_DPP_ROW_ROR8>(__float_as_int(m)));
    m = p > m ? p : m;
    const float m0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(m), 0));
    const float m1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(m), 16));
    return m1 > m0 ? m1 : m0;
}
__device__ __forceinline__ int mv_sum32(int v) {
    v = qmh_sum8(v);
    v += qmh_dpp<MV_DPP_ROW_ROR8>(v);
    return __builtin_amdgcn_readlane(v, 0) + __builtin_amdgcn_readlane(v, 16);
}

// y: the row's result. Lanes of one tile hold consecutive rows, so the RoPE partner of row
// 2i/2i+1 is lane ^ 1 and the W3 partner of an interleaved W1 row is lane + R/2.
// K goes to a transposed cache [kvd][max_seq], V to a row cache [max_seq][kvd].
// half: R/2 of the tile (the SwiGLU epilogues; 32 for SWIGLU_Q)
__device__ __forceinline__ void mv_epilogue(const qmh_mv_args &a, int row, float y, int lane, int half, int pos,
                                            const EpiIn &e, const uint64_t *etab) {
    switch (a.epi) {
    case QMH_EPI_STORE:
        if (row < a.rows) a.out0[row] = y;
        break;
    case QMH_EPI_ADD:  // x[i] += y[i] (src/model.c:179,186)
        if (row < a.rows) a.out0[row] = e.resid + y;
        break;
    case QMH_EPI_QKV: {
        const float partner = __shfl_xor(y, 1);
        // the position comes from device memory: never let a stale one address past the cache
        if (row >= a.rows || pos < 0 || pos >= a.max_seq) break;
        if (row < a.seg2) {  // q or k: rotate the (2i, 2i+1) pair, src/ops.c:114-126
            const int local = row < a.seg1 ? row : row - a.seg1;
            const float v = (local & 1) == 0 ? (y * e.c - partner * e.s) : (partner * e.s + y * e.c);
            if (row < a.seg1) a.out0[local] = v;
            else a.out1[(size_t)local * a.max_seq + pos] = v;
        } else {
            a.out2[(size_t)pos * a.kvd + (row - a.seg2)] = y;
        }
        break;
    }
    case QMH_EPI_SWIGLU: {  // silu(g)*u (src/ops.c:128-133)
        const float up = __shfl_down(y, half);
        if (lane < half && row < a.rows) a.out0[row] = y / (1.0f + qmh_expf_t(-y, etab)) * up;
        break;
    }
    case QMH_EPI_SWIGLU_Q: {  // R == 64: lanes 0..31 hold the block (rows 32*b ..), 0 past rows
        // the W3 row of lane l (< 32) is lane l + 32: lanes 32..63 swapped into 0..31
        const float up = __uint_as_float(
            __builtin_amdgcn_permlane32_swap(__float_as_uint(y), __float_as_uint(y), false, false)[1]);
        const bool mine = lane < 32 && row < a.rows;
        const float h = mine ? y / (1.0f + qmh_expf_t(-y, etab)) * up : 0.0f;
        if (mine && a.out0) a.out0[row] = h;
        // the next matvec's activation block, as qm_quantize_row_q8 makes it (src/quant.c:55-63):
        // its amax starts at 0 and takes a value only when greater, so a NaN never counts
        const float ah = fabsf(h);
        const float m = mv_amax32(ah > 0.0f ? ah : 0.0f);
        const uint16_t dh = qmh_f2h(qmh_div127(m));
        const float dd = qmh_h2f(dh);
        const int q = qmh_q8_code_fast(h, dd, qmh_rcp(dd));
        const int qs = mv_sum32(q);
        if (lane < 32) {
            const int b = (row - lane) >> 5;
            uint8_t *img = (uint8_t *)a.xq_img;
            const int at = a.xq_split ? ((lane & 1) ? 16 + (lane >> 1) : (lane >> 1)) : lane;
            img[(size_t)b * 32 + at] = (uint8_t)(int8_t)q;
            if (lane == 0) {
                ((float *)(img + (size_t)a.xq_nb * 32))[b] = dd;
                ((int *)(img + (size_t)a.xq_nb * 36))[b] = qs;
            }
        }
        break;
    }
    }
}

// activation modes of k_matvec: quantize x (optionally RMSNorm'd first), or copy a quantized
// image another kernel wrote (QMH_XQ_IMAGE_BYTES layout)
enum { MV_ACT = 0, MV_ACT_NORM = 1, MV_ACT_IMAGE = 2 };
// uint4 per thread for an image of up to CAP bytes: 16 KiB (nb <= 409) in the instance every
// matvec of the 7B shapes shares, 40 KiB (nb <= 1024: hidden_dim <= 32768, the W2 input of the
// 13B / Mistral-7B / Llama-3-8B / 70B feed-forward widths 13824, 14336 and 28672) in a second
// instance that only rows past 16 KiB of image launch (a third register set in the shared instance
// cost its W2 1%, measured)
#define QMH_MV_IMAGE_CAP 16384
#define QMH_MV_IMAGE_CAP_WIDE 40960
template <int NT, int CAP = QMH_MV_IMAGE_CAP>
struct ImageRegs {
    static constexpr int N = (CAP + 16 * NT - 1) / (16 * NT);
};

#ifndef QMH_MV_D
#define QMH_MV_D 2  // chunks in flight per workgroup
#endif
// Timed on MI355X over the 7B shapes: 512 threads x 2 chunks x 2 Q4 slots (32 KiB of weights in
// flight per workgroup) beat 256 threads x 4 slots by 6-20%, and every deeper or wider variant
#ifndef QMH_MV_CH
#define QMH_MV_CH 2  // Q4_0 slots per thread per chunk (Q8_0: half)
#endif
#ifndef QMH_MV_NT
#define QMH_MV_NT 512  // threads per workgroup
#endif

// ============================================================================ quantized matvec
//
// y = W x with W Q4_0 or Q8_0 and x quantized to Q8_0 (src/ops.c:36-61), one row's dot as in
// src/kernels_scalar.c:12-34:  s = +0; for b: s = s + (float)acc_b * (d_w,b * d_x,b).
// acc_b, the int32 dot of one block, is exact in any order (sdot4); the float steps keep the
// reference's order: each term t_b = (float)acc_b * (d_w*d_x) is rounded as the reference
// rounds it, and each row's terms are summed by one lane in block order.
//
// Layout of the work, for bandwidth and few instructions per block:
//   * about one workgroup per CU, each owning a contiguous range of whole tiles (contiguous
//     slots), streamed as chunks of 256*CH slots through a ring of D register buffers: the
//     activation prologue runs under the first D chunks, and only the range's last chunk is
//     partial;
//   * buffer loads with a per-lane byte offset fixed for the whole kernel; each load's
//     resource starts at its 256 slots (scalar arithmetic), and the hardware range check
//     zeroes slots past the range without a memory access;
//   * the activation in LDS as 48-byte records (32 codes, d, code sum), laid out unrolled:
//     record j holds block j mod nb for j < nb + CHUNK/R, so a chunk's records are a scalar
//     base plus a per-lane constant and nothing wraps (no vector work between a chunk's
//     arrival and the next chunk's loads);
//   * the terms in LDS row-contiguous (each row's nb terms in block order, rows padded to
//     mv_term_stride floats): a lane's term stores advance by a fixed block step (its row never
//     changes), and after the last chunk every row's serial chain reads its terms as float4s
//     (qmh_chain_lds; W2's 344-term chains went 9.18 -> 8.24 us against 4-byte reads at stride
//     R), then the epilogue.
// Each workgroup quantizes the activation once for all of its rows.
constexpr int MV_REC = 48;  // LDS bytes per activation record

// first tile of workgroup w of G over ntiles (w * ntiles < 2^32 for every launch: 32-bit division,
// which the kernel's start waits for)
__host__ __device__ __forceinline__ int mv_tile0(int w, int ntiles, int G) {
    return (int)((unsigned)w * (unsigned)ntiles / (unsigned)G);
}
__host__ __device__ __forceinline__ int mv_nrec(int nb, int R, int chq4, int dtype_q4, int nt) {
    return nb + nt * (dtype_q4 ? chq4 : chq4 / 2) / R;
}
// LDS row stride (floats) of the terms: a row's nb terms contiguous, rounded up to whole float4s,
// plus 4 so that rows r and r+1 start 4 banks apart
__host__ __device__ __forceinline__ int mv_term_stride(int nb) { return ((nb + 3) & ~3) + 4; }
// dynamic LDS bytes of k_matvec: the records, then T for up to `tiles` tiles
__host__ __device__ __forceinline__ size_t mv_lds_bytes(int nb, int R, int tiles, int chq4, int dtype_q4, int nt) {
    return (size_t)mv_nrec(nb, R, chq4, dtype_q4, nt) * MV_REC + 4 * (size_t)tiles * R * mv_term_stride(nb);
}

typedef unsigned int mv_u32x4 __attribute__((ext_vector_type(4)));
// cache policy of the weight loads: non-temporal (each weight byte is read once per token), so the
// stream does not evict the code, the activations and the norm gains from L2 (timed on MI355X:
// 585 -> 591 tok/s at c5a)
#define MV_NT 2

// One instance per weight type serves every matvec of the token (tile height R and activation
// mode are uniform runtime values): the decode step's kernels then share one copy of this code in
// the instruction cache, instead of refetching a different instance's code (from HBM, the
// weight stream having evicted it from L2) at every launch.
template <int WT, int D, int CHQ4, int NT, int ICAP = QMH_MV_IMAGE_CAP>
__global__ __launch_bounds__(NT) void k_matvec(qmh_mv_args a) {
    constexpr int CB = WT == QMH_Q4 ? 16 : 32;           // code bytes per block
    constexpr int NV = CB / 16;                          // uint4 per block
    constexpr int CH = WT == QMH_Q4 ? CHQ4 : CHQ4 / 2;   // slots per thread per chunk
    constexpr int CHUNK = NT * CH;
    constexpr int PX = ActRegs<false, NT>::P > ActRegs<true, NT>::P ? ActRegs<false, NT>::P : ActRegs<true, NT>::P;
    extern __shared__ __align__(16) uint8_t smem[];
    __shared__ double red[16];
    __shared__ uint64_t etab[32];  // expf's table for the SwiGLU epilogues

    // R (8, 16, 32 or 64: divides 64, so a chunk holds whole block columns) and the activation
    // mode, both uniform
    const int R = a.tile_r, lgR = __builtin_ctz((unsigned)R);
    const int am = a.xq_in ? MV_ACT_IMAGE : a.norm_w ? MV_ACT_NORM : MV_ACT;
    const int nb = a.nb, TB = R * nb, SP = mv_term_stride(nb), tid = threadIdx.x;
    const int t0 = mv_tile0(blockIdx.x, a.ntiles, gridDim.x), t1 = mv_tile0(blockIdx.x + 1, a.ntiles, gridDim.x);
    const int ntw = t1 - t0, nslot = ntw * TB, nch = (nslot + CHUNK - 1) / CHUNK;
    if (ntw <= 0) return;  // the host launches at most ntiles workgroups
    const int nrec = nb + (CHUNK >> lgR);
    float *T = (float *)(smem + (size_t)nrec * MV_REC);

    // 1. activation (or image) loads, issued first so waiting for them never waits for weights
    float4 xr[2 * PX], wr[2 * ActRegs<true, NT>::P];
    uint4 im[ImageRegs<NT, ICAP>::N];
    const int nimg = (int)(QMH_XQ_IMAGE_BYTES(nb) / 16);
    if (am == MV_ACT_IMAGE) {
        const uint4 *src = (const uint4 *)a.xq_in;
#pragma unroll
        for (int k = 0; k < ImageRegs<NT, ICAP>::N; k++)
            if (k * NT < nimg) {
                const int i = k * NT + tid;
                im[k] = src[i < nimg ? i : nimg - 1];
            }
    } else if (am == MV_ACT_NORM) {
        act_load<true, NT>(a, xr, wr);
    } else {
        act_load<false, NT>(a, xr, wr);
    }
    const int pos = a.pos_ptr ? *a.pos_ptr : 0;
    // expf's table for the SwiGLU epilogues: loaded now, stored to LDS after the stream (a store
    // here would wait for every load issued so far, the activation's included)
    const bool swiglu = a.epi == QMH_EPI_SWIGLU || a.epi == QMH_EPI_SWIGLU_Q;
    uint64_t etv = 0;
    if (swiglu && tid < 32) etv = qmh_exp2_tab[tid];

    // 2. the first D chunks. Each load's resource starts at its own 256 slots and holds what is
    // left of the range, so the range check (on the lane's offset) zeroes slots past the range
    // without touching memory; the resources are scalar arithmetic.
    const uint8_t *cbase = (const uint8_t *)a.codes + (size_t)t0 * TB * CB;
    const uint8_t *sbase = (const uint8_t *)(a.scales + (size_t)t0 * TB);
    mv_u32x4 C[D][CH][NV];
    uint32_t Sc[D][CH];
#define MV_LOAD(J, CHK)                                                                          \
    _Pragma("unroll") for (int k = 0; k < CH; k++) {                                              \
        const int so = (CHK) * CHUNK + k * NT, left = nslot - so > 0 ? nslot - so : 0;        \
        const __amdgpu_buffer_rsrc_t rc = __builtin_amdgcn_make_buffer_rsrc(                      \
            (void *)(cbase + (size_t)so * CB), (short)0, left * CB, 0x00020000);                  \
        const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(                      \
            (void *)(sbase + (size_t)so * 2), (short)0, left * 2, 0x00020000);                    \
        _Pragma("unroll") for (int v = 0; v < NV; v++) C[J][k][v] =                               \
            __builtin_amdgcn_raw_buffer_load_b128(rc, tid * CB + 16 * v, 0, MV_NT);               \
        Sc[J][k] = __builtin_amdgcn_raw_buffer_load_b16(rs, tid * 2, 0, MV_NT);                   \
    }
#pragma unroll
    for (int j = 0; j < D; j++) MV_LOAD(j, j);


    // 3. the activation records
    if (am == MV_ACT_IMAGE) {
        // global image: codes [nb][32], then d [nb], then code sums [nb] (QMH_XQ_IMAGE_BYTES)
#pragma unroll
        for (int k = 0; k < ImageRegs<NT, ICAP>::N; k++) {
            const int i = k * NT + tid;
            if (k * NT < nimg && i < nimg) {
                const int o = 16 * i;
                if (o < nb * 32) {
                    for (int rb = o / 32; rb < nrec; rb += nb)
                        *(uint4 *)(smem + rb * MV_REC + (o & 31)) = im[k];
                } else {
                    const uint32_t w4[4] = {im[k].x, im[k].y, im[k].z, im[k].w};
#pragma unroll
                    for (int w = 0; w < 4; w++) {
                        const int ow = o + 4 * w;
                        const int isd = ow < nb * 36, b = isd ? (ow - nb * 32) / 4 : (ow - nb * 36) / 4;
                        if (ow < nb * 40)
                            for (int rb = b; rb < nrec; rb += nb)
                                *(uint32_t *)(smem + rb * MV_REC + (isd ? 32 : 36)) = w4[w];
                    }
                }
            }
        }
        __syncthreads();
    } else {
        const ActDst dst{(int8_t *)smem, MV_REC, (float *)(smem + 32), (int *)(smem + 36), MV_REC / 4, nrec};
        if (am == MV_ACT_NORM) act_finish<WT == QMH_Q4, true, NT>(a, xr, wr, dst, red);
        else act_finish<WT == QMH_Q4, false, NT>(a, xr, wr, dst, red);
    }

    // the first row group's epilogue inputs, issued after the activation records: issued behind the
    // first chunks, a load the prologue does not wait for made its waits for the activation wait for
    // the first weights too (the wait counts cover every path, and the load is conditional)
    const int rows_w = ntw * R;
    EpiIn ein = {0.0f, 1.0f, 0.0f};
    if (tid < rows_w) {
        const int tile = t0 + (tid >> lgR), r = tid & (R - 1);
        ein = epi_fetch(a, R >= 2 * QMH_TILE_R ? tile * (R / 2) + (r & (R / 2 - 1)) : tile * R + r, pos);
    }

    // 4. the stream. Thread tid's slot k of chunk c is l = c*CHUNK + k*NT + tid: block column
    // (l / R) = c*CHUNK/R + k*NT/R + tid/R, record (that mod nb) = um + k*NT/R + tid/R in the
    // unrolled layout, with um = (c*CHUNK/R) mod nb.
    const uint8_t *rec_t = smem + (tid >> lgR) * MV_REC;
    const int ntr = NT >> lgR;  // block columns per NT slots
    // the terms sit row-contiguous: term (tile tl, block b, row r) at T[(tl*R + r)*SP + b]. A
    // thread's slots advance by NT per term (k, then chunk), so its block column advances by ntr:
    // (tl, b) is carried along, and its row r = tid % R never changes
    int tw = 0, bw = tid >> lgR;
    while (bw >= nb) bw -= nb, tw++;
    float *T_r = T + (tid & (R - 1)) * SP;
#define MV_COMPUTE(J, CHK, UM, CHECK)                                                                   \
    _Pragma("unroll") for (int k = 0; k < CH; k++) {                                                     \
        const uint8_t *rp = rec_t + ((UM) + k * ntr) * MV_REC;                                           \
        const int4 x0 = *(const int4 *)rp, x1 = *(const int4 *)(rp + 16);                                \
        const float2 ds = *(const float2 *)(rp + 32);                                                    \
        int acc;                                                                                         \
        if (WT == QMH_Q4) {                                                                              \
            const mv_u32x4 w = C[J][k][0];                                                              \
            acc = -8 * __float_as_int(ds.y); /* sum (q-8)*x = sum q*x - 8*sum x, exact */                \
            acc = __builtin_amdgcn_sdot4((int)(w.x & 0x0f0f0f0fu), x0.x, acc, false);                    \
            acc = __builtin_amdgcn_sdot4((int)((w.x >> 4) & 0x0f0f0f0fu), x1.x, acc, false);             \
            acc = __builtin_amdgcn_sdot4((int)(w.y & 0x0f0f0f0fu), x0.y, acc, false);                    \
            acc = __builtin_amdgcn_sdot4((int)((w.y >> 4) & 0x0f0f0f0fu), x1.y, acc, false);             \
            acc = __builtin_amdgcn_sdot4((int)(w.z & 0x0f0f0f0fu), x0.z, acc, false);                    \
            acc = __builtin_amdgcn_sdot4((int)((w.z >> 4) & 0x0f0f0f0fu), x1.z, acc, false);             \
            acc = __builtin_amdgcn_sdot4((int)(w.w & 0x0f0f0f0fu), x0.w, acc, false);                    \
            acc = __builtin_amdgcn_sdot4((int)((w.w >> 4) & 0x0f0f0f0fu), x1.w, acc, false);             \
        } else {                                                                                         \
            const mv_u32x4 w0 = C[J][k][0], w1 = C[J][k][NV - 1];                                       \
            acc = __builtin_amdgcn_sdot4((int)w0.x, x0.x, 0, false);                                     \
            acc = __builtin_amdgcn_sdot4((int)w0.y, x0.y, acc, false);                                   \
            acc = __builtin_amdgcn_sdot4((int)w0.z, x0.z, acc, false);                                   \
            acc = __builtin_amdgcn_sdot4((int)w0.w, x0.w, acc, false);                                   \
            acc = __builtin_amdgcn_sdot4((int)w1.x, x1.x, acc, false);                                   \
            acc = __builtin_amdgcn_sdot4((int)w1.y, x1.y, acc, false);                                   \
            acc = __builtin_amdgcn_sdot4((int)w1.z, x1.z, acc, false);                                   \
            acc = __builtin_amdgcn_sdot4((int)w1.w, x1.w, acc, false);                                   \
        }                                                                                                \
        const float t = (float)acc * (qmh_h2f((uint16_t)Sc[J][k]) * ds.x);                               \
        if (!(CHECK) || (CHK) * CHUNK + k * NT + tid < nslot) T_r[tw * R * SP + bw] = t;           \
        bw += ntr;                                                                                       \
        while (bw >= nb) bw -= nb, tw++;                                                                 \
    }

    int c0 = 0, um = 0;  // um: record of the chunk's first block column
    const int ustep = (CHUNK >> lgR) % nb;
    for (; c0 + D < nch; c0 += D) {
#pragma unroll
        for (int j = 0; j < D; j++) {
            MV_COMPUTE(j, c0 + j, um, false);
            MV_LOAD(j, c0 + j + D);
            um += ustep;
            um -= um >= nb ? nb : 0;
        }
    }
#pragma unroll
    for (int j = 0; j < D; j++)
        if (c0 + j < nch) {
            MV_COMPUTE(j, c0 + j, um, true);
            um += ustep;
            um -= um >= nb ? nb : 0;
        }
#undef MV_COMPUTE
#undef MV_LOAD
    if (swiglu && tid < 32) etab[tid] = etv;
    __syncthreads();

    // 5. serial chains (row i of the range: tile i/R, row i%R; its terms at T[i*SP ..]) and
    // epilogues; a wave holds whole tiles (R divides 64, or R == 64)
    for (int i0 = 0; i0 < rows_w; i0 += NT) {
        const int i = i0 + tid;
        if (i0 + (tid & ~63) >= rows_w) break;  // the whole wave is past the range
        const int tl = i >> lgR, r = i & (R - 1), tile = t0 + tl;
        const int row = R >= 2 * QMH_TILE_R ? tile * (R / 2) + (r & (R / 2 - 1)) : tile * R + r;
        const bool mine = i < rows_w;
        if (i0 > 0 && mine) ein = epi_fetch(a, row, pos);
        float y = 0.0f;
        if (mine) y = qmh_chain_lds(T + (size_t)(tl * R + r) * SP, nb, 0.0f);
        mv_epilogue(a, mine ? row : a.rows, y, r, R >> 1, pos, ein, etab);
    }
}

// f32 weights (src/kernels_scalar.c:6-10 via src/ops.c:42-45): s = +0; s = s + w_i*x_i in index
// order, one lane per row. A workgroup owns MF_R consecutive rows and has MF_NL loader threads plus
// one chain wave. The weights stream in chunks of MF_C columns, coalesced (64 consecutive loader
// threads read 1 KB of one row), two chunks ahead in registers. The loaders turn a chunk into its
// products w_i*x_i (the reference's multiply, rounded alone) and stage them in LDS, one of two
// buffers, while the chain wave's first MF_R lanes add the previous chunk's products in index
// order, 32 per step, with the next 32 already read from LDS. The activation (RMSNorm'd when a gain
// is given, as the reference's (x*inv)*w) sits in LDS for every chunk. One barrier per chunk. The
// chains bound the kernel: a dependent add fed from LDS takes ~10 clocks, so 4096 columns ~17 us.
#define MF_R 16
#define MF_C 256
#define MF_NL 512                         // loader threads (waves 0-7); wave 8 runs the chains
#define MF_NT (MF_NL + 64)
#define MF_L4 (MF_R * MF_C / 4 / MF_NL)  // float4 loads per loader thread per chunk
__global__ __launch_bounds__(MF_NT) void k_matvec_f32(qmh_mv_args a) {
    static_assert(MF_L4 * MF_NL * 4 == MF_R * MF_C && MF_C % 64 == 0 && MF_R <= 64, "whole float4 chunks");
    constexpr int TS = MF_C + 4;  // LDS row stride of a chunk (== 4 mod 64 floats)
    extern __shared__ __align__(16) uint8_t smem[];
    __shared__ double red[16];
    float *xs = (float *)smem;                                    // [cols rounded up to MF_C]
    const int n = a.cols, nch = (n + MF_C - 1) / MF_C, tid = threadIdx.x;
    const bool loader = tid < MF_NL, chain = tid >= MF_NL && tid < MF_NL + MF_R;
    float *tile = xs + (size_t)nch * MF_C;                        // [2][MF_R][TS] products
    const int r0 = blockIdx.x * MF_R;
    // chunk c's loads: float4 f = k*MF_NL + tid is row f / (MF_C/4), columns 4*(f % (MF_C/4)) ..; rows
    // past the matrix re-read its last row, columns past n read the row's last whole float4 (or,
    // for n % 4 != 0, element by element); the chains stop at n, so those products are never added
    const float *W = (const float *)a.codes;
    float4 ld[2][MF_L4];
    auto issue = [&](int c, float4(&d)[MF_L4]) {
#pragma unroll
        for (int k = 0; k < MF_L4; k++) {
            const int f = k * MF_NL + tid, rr = f / (MF_C / 4), col = c * MF_C + 4 * (f % (MF_C / 4));
            const int row = r0 + rr < a.rows ? r0 + rr : a.rows - 1;
            const float *wr = W + (size_t)row * n;
            if ((n & 3) == 0) {
                d[k] = qmh_ld_nt4(wr + (col <= n - 4 ? col : n - 4));
            } else {
                float v[4];
#pragma unroll
                for (int j = 0; j < 4; j++) v[j] = wr[col + j < n ? col + j : n - 1];
                d[k] = make_float4(v[0], v[1], v[2], v[3]);
            }
        }
    };
    // chunk c's products into buffer t (xs is zero past n)
    auto stash = [&](int c, const float4(&d)[MF_L4], float *t) {
#pragma unroll
        for (int k = 0; k < MF_L4; k++) {
            const int f = k * MF_NL + tid, c4 = 4 * (f % (MF_C / 4));
            const float4 x4 = *(const float4 *)(xs + (size_t)c * MF_C + c4);
            float4 p;
            p.x = d[k].x * x4.x;
            p.y = d[k].y * x4.y;
            p.z = d[k].z * x4.z;
            p.w = d[k].w * x4.w;
            *(float4 *)(t + (f / (MF_C / 4)) * TS + c4) = p;
        }
    };
    if (loader) {
        issue(0, ld[0]);
        if (nch > 1) issue(1, ld[1]);
    }
    // the activation, normalised as the reference does when a gain is given (src/ops.c:93-98)
    float inv = 1.0f;
    if (a.norm_w) {
        double ss = 0.0;
        for (int i = tid; i < n; i += MF_NT) {
            const double v = (double)a.x[i];
            ss += v * v;
        }
        ss = qmh_block_sum_d(ss, red);
        const double d = qmh_sum_slack(ss, n);
        inv = qmh_rms_inv(ss - d, n, a.eps);
        if (inv != qmh_rms_inv(ss + d, n, a.eps)) {  // uniform; serial sum as the reference
            if (tid == 0) {
                double sr = 0.0;
                for (int i = 0; i < n; i++) sr += (double)a.x[i] * (double)a.x[i];
                red[15] = sr;
            }
            __syncthreads();
            inv = qmh_rms_inv(red[15], n, a.eps);
        }
    }
    for (int i = tid; i < nch * MF_C; i += MF_NT)
        xs[i] = i < n ? (a.norm_w ? a.x[i] * inv * a.norm_w[i] : a.x[i]) : 0.0f;
    __syncthreads();
    if (loader) {
        stash(0, ld[0], tile);
        if (nch > 2) issue(2, ld[0]);
    }
    __syncthreads();
    float s = 0.0f;
    // step c: the chains add chunk c from buffer c % 2 while the loaders stage chunk c+1 (registers
    // ld[(c+1) % 2]) into buffer (c+1) % 2 and refill those registers with chunk c+3 (unrolled by
    // two: the register sets are indexed statically)
    auto step = [&](int c, float4(&nxt)[MF_L4]) {
        const int b = c & 1;
        if (chain) {
            const float *pr = tile + (size_t)b * MF_R * TS + (size_t)(tid - MF_NL) * TS;
            const int m = n - c * MF_C < MF_C ? n - c * MF_C : MF_C;
            if (m == MF_C) {
                // 32 products per read set from two register sets: the reads of set st+1 go out
                // before the adds of set st (the scheduling barriers keep them there), so each
                // set waits only for reads issued a set earlier
                const float4 *p4 = (const float4 *)pr;
                float4 A[8], B[8];
                auto rd = [&](float4(&d)[8], int st) {
#pragma unroll
                    for (int q = 0; q < 8; q++) d[q] = p4[8 * st + q];
                };
                auto add = [&](const float4(&d)[8]) {
#pragma unroll
                    for (int q = 0; q < 8; q++) {
                        s = s + d[q].x;
                        s = s + d[q].y;
                        s = s + d[q].z;
                        s = s + d[q].w;
                    }
                };
                rd(A, 0);
#pragma unroll 1
                for (int st = 0; st < MF_C / 32; st += 2) {
                    rd(B, st + 1);
                    __builtin_amdgcn_sched_barrier(0);
                    add(A);
                    __builtin_amdgcn_sched_barrier(0);
                    rd(A, st + 2 < MF_C / 32 ? st + 2 : st);  // the last pair re-reads a set: no branch
                    __builtin_amdgcn_sched_barrier(0);
                    add(B);
                    __builtin_amdgcn_sched_barrier(0);
                }
            } else {  // the last chunk, ragged
                for (int j = 0; j < m; j++) s = s + pr[j];
            }
        }
        if (loader && c + 1 < nch) {
            stash(c + 1, nxt, tile + (size_t)(b ^ 1) * MF_R * TS);
            if (c + 3 < nch) issue(c + 3, nxt);
        }
        __syncthreads();
    };
    for (int c = 0; c < nch; c += 2) {
        step(c, ld[1]);
        if (c + 1 < nch) step(c + 1, ld[0]);
    }
    // the chain wave's lanes hold rows r0 + lane (lane < MF_R)
    const int lane = tid & 63, row = r0 + (lane & (MF_R - 1));
    const int pos = a.pos_ptr ? *a.pos_ptr : 0;
    if (tid >= MF_NL) {
        const EpiIn e = epi_fetch(a, row, pos);
        mv_epilogue(a, lane < MF_R ? row : a.rows, s, lane & (MF_R - 1), MF_R, pos, e, qmh_exp2_tab);
    }
}

extern "C" int qmh_matvec_max_cols(int norm) {
    return (norm ? ActRegs<true, QMH_MV_NT>::P : ActRegs<false, QMH_MV_NT>::P) * QMH_MV_NT * 8;
}

// the longest row whose input comes as a quantized image (QMH_XQ_IMAGE_BYTES(nb) <= the image registers)
extern "C" int qmh_matvec_max_image_cols(void) {
    return (ImageRegs<QMH_MV_NT, QMH_MV_IMAGE_CAP_WIDE>::N * QMH_MV_NT * 16) / 40 * 32;
}

// Workgroups for k_matvec: `want` (about one per CU; more for matrices of many tiles), never
// more than ntiles, and enough that a workgroup's records and terms fit the 64 KiB of LDS one
// workgroup may take. -1: one tile does not fit.
// LDS budgets of a k_matvec workgroup: 64 KiB, or where one tile's records and terms do not fit
// that (rows of more than ~7000 columns in 64-row tiles, W2's input past ~13000), up to 152 KiB
// (one workgroup per CU either way; the 7B shapes' grids are those of the 64 KiB budget)
#define MV_LDS 65536
#define MV_LDS_WIDE (152 * 1024)
extern "C" int qmh_matvec_grid(int ntiles, int nb, int tile_r, int dtype, int want) {
    if (ntiles < 1 || nb < 1 || (dtype != QMH_Q4 && dtype != QMH_Q8)) return -1;
    const size_t rec = (size_t)mv_nrec(nb, tile_r, QMH_MV_CH, dtype == QMH_Q4, QMH_MV_NT) * MV_REC;
    const size_t per = 4 * (size_t)tile_r * mv_term_stride(nb);
    const size_t budget = rec + per <= MV_LDS ? MV_LDS : MV_LDS_WIDE;
    if (rec + per > budget) return -1;
    const int maxt = (int)((budget - rec) / per);
    int g = want < ntiles ? want : ntiles;
    const int need = (ntiles + maxt - 1) / maxt;
    return g > need ? g : need;
}

extern "C" int qmh_launch_matvec(const qmh_mv_args *a, int grid, void *stream) {
    const bool norm = a->norm_w != NULL, image = a->xq_in != NULL;
    if (a->tile_r != 8 && a->tile_r != 16 && a->tile_r != 32 && a->tile_r != 64) return (int)hipErrorInvalidValue;
    if (a->epi == QMH_EPI_SWIGLU && a->tile_r < 32) return (int)hipErrorInvalidValue;  // interleaved W1|W3 tiles
    // an image input is bounded by the image registers (checked below), a float input by ActRegs
    if (grid < 1 || grid > a->ntiles || a->cols < 1 || (!image && a->cols > qmh_matvec_max_cols(norm)) || (norm && image) ||
        (unsigned long long)grid * (unsigned long long)a->ntiles >= (1ull << 32))  // mv_tile0's 32-bit product
        return (int)hipErrorInvalidValue;
    if (a->dtype != QMH_Q4 && a->dtype != QMH_Q8) return (int)hipErrorInvalidValue;
    const int tmax = (a->ntiles + grid - 1) / grid;
    const size_t lds = mv_lds_bytes(a->nb, a->tile_r, tmax, QMH_MV_CH, a->dtype == QMH_Q4, QMH_MV_NT);
    if (lds > MV_LDS_WIDE || (long long)tmax * a->tile_r * a->nb * (a->dtype == QMH_Q4 ? 16 : 32) >= (1ll << 31))
        return (int)hipErrorInvalidValue;
    if (image && QMH_XQ_IMAGE_BYTES(a->nb) > (size_t)ImageRegs<QMH_MV_NT, QMH_MV_IMAGE_CAP_WIDE>::N * QMH_MV_NT * 16)
        return (int)hipErrorInvalidValue;
    const bool wide = image && QMH_XQ_IMAGE_BYTES(a->nb) > (size_t)ImageRegs<QMH_MV_NT>::N * QMH_MV_NT * 16;
    if ((a->epi == QMH_EPI_SWIGLU_Q) != (a->tile_r == 64)) return (int)hipErrorInvalidValue;
    hipStream_t s = (hipStream_t)stream;
    if (wide && a->dtype == QMH_Q4)
        hipLaunchKernelGGL((k_matvec<QMH_Q4, QMH_MV_D, QMH_MV_CH, QMH_MV_NT, QMH_MV_IMAGE_CAP_WIDE>), dim3(grid),
                           dim3(QMH_MV_NT), lds, s, *a);
    else if (wide)
        hipLaunchKernelGGL((k_matvec<QMH_Q8, QMH_MV_D, QMH_MV_CH, QMH_MV_NT, QMH_MV_IMAGE_CAP_WIDE>), dim3(grid),
                           dim3(QMH_MV_NT), lds, s, *a);
    else if (a->dtype == QMH_Q4)
        hipLaunchKernelGGL((k_matvec<QMH_Q4, QMH_MV_D, QMH_MV_CH, QMH_MV_NT>), dim3(grid), dim3(QMH_MV_NT), lds, s, *a);
    else
        hipLaunchKernelGGL((k_matvec<QMH_Q8, QMH_MV_D, QMH_MV_CH, QMH_MV_NT>), dim3(grid), dim3(QMH_MV_NT), lds, s, *a);
    return (int)hipGetLastError();
}

// dynamic LDS of k_matvec_f32: the activation rounded up to whole chunks, then two chunks
static size_t mf_lds_bytes(int cols) {
    return sizeof(float) * ((size_t)(cols + MF_C - 1) / MF_C * MF_C + 2 * (size_t)MF_R * (MF_C + 4));
}

extern "C" int qmh_launch_matvec_f32(const qmh_mv_args *a, void *stream) {
    if (a->rows < 1 || a->cols < 1 || mf_lds_bytes(a->cols) > 160 * 1024 - 1024) return (int)hipErrorInvalidValue;
    const int grid = (a->rows + MF_R - 1) / MF_R;
    hipLaunchKernelGGL(k_matvec_f32, dim3(grid), dim3(MF_NT), mf_lds_bytes(a->cols), (hipStream_t)stream, *a);
    return (int)hipGetLastError();
}
