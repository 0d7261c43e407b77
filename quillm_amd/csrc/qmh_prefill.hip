// gfx950 batched prefill: P prompt tokens through the model at once, bitwise equal to P
// sequential forwards (the reference's prompt loop, src/main.c:127-130, calling
// qm_model_forward, src/model.c:158-191).
//
// Exactness, layer by layer:
//   * activations are quantized per token row exactly as qm_quantize_row_q8 does (src/quant.c);
//   * a matmul row (r, token p) is the reference's serial chain s = +0; s = s + (float)acc_b *
//     (dw_b * dx_b) over blocks b in order (src/kernels_scalar.c:12-34). acc_b, the exact int32
//     dot of one 32-element block, comes from one v_mfma_i32_16x16x32_i8 with a zero
//     accumulator (16 rows x 16 tokens x one block per instruction); each lane then extends the
//     float chains of its 4 (row, token) pairs;
//   * attention scores, softmax and the weighted V sum keep the decode kernels' per-element
//     orders (serial over head_dim, the reference softmax, serial over positions).
//
// MFMA operand layout (v_mfma_i32_16x16x32_i8, checked on the device): A[i][k] in lane
// i + 16*(k/8), byte k%8; B[k][j] in lane j + 16*(k/8), byte k%8; D[i][j] in lane j + 16*(i/4),
// element i%4. Any permutation of k applied to both operands leaves the dot unchanged; for
// Q4_0 weights each 8-element group is taken as [e0 e2 e4 e6 e1 e3 e5 e7] (the low nibbles of
// 4 bytes, then the high nibbles), and activations are stored in the same order.
#include "qmh_device.h"
#include "qmh_launch.h"

#define QMH_Q8 2
#define QMH_Q4 3

typedef int pf_v4i __attribute__((ext_vector_type(4)));
typedef float pf_v4f __attribute__((ext_vector_type(4)));
typedef _Float16 pf_v4h __attribute__((ext_vector_type(4)));

// ============================================================================ embedding

__global__ void k_pf_embed(const uint8_t *__restrict__ E, int dtype, int dim, int vocab, const int32_t *tokens,
                           float *X) {
    const int p = blockIdx.x;
    int tok = tokens[p];
    tok = tok < 0 ? 0 : (tok >= vocab ? vocab - 1 : tok);  // the host validated the ids
    const size_t nbr = (size_t)(dim + 31) / 32;
    float *xr = X + (size_t)p * dim;
    if (dtype == QMH_Q8 || dtype == QMH_Q4) {
        // a quarter block (8 values) per thread: the scale, then the codes as 16-bit loads (a block's
        // codes start 2 bytes in, so they are only 2-byte aligned)
        const int bs = dtype == QMH_Q8 ? 34 : 18;
        for (int g = threadIdx.x; g < (int)nbr * 4; g += blockDim.x) {
            const int b = g >> 2, k0 = (g & 3) * 8;
            if (b * 32 + k0 >= dim) continue;
            const uint8_t *blk = E + ((size_t)tok * nbr + b) * bs;
            const float d = qmh_h2f(*(const uint16_t *)blk);
            float v[8];
            if (dtype == QMH_Q8) {
                const uint16_t *c = (const uint16_t *)(blk + 2 + k0);
#pragma unroll
                for (int h = 0; h < 4; h++) {
                    const uint16_t w = c[h];
                    v[2 * h] = d * (float)(int8_t)(w & 0xff);
                    v[2 * h + 1] = d * (float)(int8_t)(w >> 8);
                }
            } else {
                const uint16_t *c = (const uint16_t *)(blk + 2 + k0 / 2);  // element k: byte k/2, low nibble first
#pragma unroll
                for (int h = 0; h < 2; h++) {
                    const uint16_t w = c[h];
#pragma unroll
                    for (int q = 0; q < 4; q++) v[4 * h + q] = d * (float)((int)((w >> (4 * q)) & 15) - 8);
                }
            }
#pragma unroll
            for (int k = 0; k < 8; k++)
                if (b * 32 + k0 + k < dim) xr[b * 32 + k0 + k] = v[k];
        }
    } else {
        for (int i = threadIdx.x; i < dim; i += blockDim.x) xr[i] = ((const float *)E)[(size_t)tok * dim + i];
    }
}

extern "C" int qmh_launch_pf_embed(const uint8_t *tok_embd, int dtype, int dim, int vocab, const int32_t *tokens,
                                   int P, float *X, void *stream) {
    hipLaunchKernelGGL(k_pf_embed, dim3(P), dim3(256), 0, (hipStream_t)stream, tok_embd, dtype, dim, vocab, tokens, X);
    return (int)hipGetLastError();
}

// ============================================================================ activation quantization
//
// Row p of x (n values, optionally RMSNorm'd with gain w: src/ops.c:93-98) -> Q8_0 blocks of the
// token-major-within-block image: codes xc[(b*PP + p)*32 + k], scales xd[b*PP + p] (fp32 of the
// fp16 d). perm8: codes of each 8-group in the order e0 e2 e4 e6 e1 e3 e5 e7 (Q4_0 consumers).
// One workgroup per token; 8 lanes per block, 4 values each, as the decode prologue.
// One thread's share of a block quantization: block b = 32*r + tid/8 (round r), values 4*(tid%8)
// .. +3 of it, as the decode prologue (amax over 8 lanes by DPP), then the codes and the scale.
__device__ __forceinline__ void pf_quant_block(const float (&v)[4], int b, int nb, int p, int sub, int8_t *xc,
                                               float *xd, int PP, int perm8) {
    float m = 0.0f;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const float av = fabsf(v[j]);
        m = av > m ? av : m;
    }
    m = qmh_amax8(m);
    const float dd = qmh_h2f(qmh_f2h(qmh_div127(m)));
    int q[4];
    qmh_q8_codes4(v, dd, qmh_rcp(dd), q);
    const uint32_t b0 = (uint32_t)q[0] & 0xffu, b1 = (uint32_t)q[1] & 0xffu, b2 = (uint32_t)q[2] & 0xffu,
                   b3 = (uint32_t)q[3] & 0xffu;
    // one dword per lane: bytes 4*sub .. +3 of the block. perm8 (elements 8g+e, e = 0..7, at
    // 8g + {0,4,1,5,2,6,3,7}[e]): the lane pair of a group (elements 0-3, 4-7) swaps half-words,
    // {e0 e2 | e1 e3} against {e4 e6 | e5 e7}, and writes {e0 e2 e4 e6} (even lane) or {e1 e3 e5 e7}.
    const uint32_t pk = b0 | (b2 << 8) | (b1 << 16) | (b3 << 24);
    const uint32_t pp = (uint32_t)qmh_dpp<QMH_DPP_QXOR1>((int)pk);  // every lane of the block is active here
    const uint32_t w = !perm8 ? (b0 | (b1 << 8) | (b2 << 16) | (b3 << 24))
                       : (sub & 1) == 0 ? ((pk & 0xffffu) | (pp << 16)) : ((pp >> 16) | (pk & 0xffff0000u));
    if (b < nb) {
        *(uint32_t *)(xc + ((size_t)b * PP + p) * 32 + 4 * sub) = w;
        if (sub == 0) xd[(size_t)b * PP + p] = dd;
    }
}

// One workgroup per token; 8 lanes per block, 4 values each. Rows of up to PQ_R*1024 values are
// loaded once into registers (one round of loads), larger ones round by round.
#define PQ_R 16
template <int NT>
__global__ __launch_bounds__(NT) void k_pf_quant(const float *__restrict__ x, int ldx, const float *w, float eps,
                                                     int n, int8_t *xc, float *xd, int PP, int perm8) {
    __shared__ double red[NT / 64 + 1];  // the waves' partial sums, then the serial sum
    const int p = blockIdx.x, tid = threadIdx.x, nb = (n + 31) / 32, sub = tid & 7;
    const int R = (nb + NT / 8 - 1) / (NT / 8);  // rounds of 32 blocks
    const float *row = x + (size_t)p * ldx;
    const bool held = R <= PQ_R;
    float xv[PQ_R][4];
    double ss = 0.0;
    if (held) {
#pragma unroll
        for (int r = 0; r < PQ_R; r++)
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int i = (r * (NT / 8) + (tid >> 3)) * 32 + sub * 4 + j;
                xv[r][j] = (r < R && i < n) ? row[i] : 0.0f;
            }
        if (w)
#pragma unroll
            for (int r = 0; r < PQ_R; r++)
#pragma unroll
                for (int j = 0; j < 4; j++) ss += (double)xv[r][j] * (double)xv[r][j];
    } else if (w) {
        for (int i = tid; i < n; i += NT) ss += (double)row[i] * (double)row[i];
    }
    float inv = 1.0f;
    if (w) {
        ss = qmh_block_sum_d(ss, red);
        const double d = qmh_sum_slack(ss, n);
        inv = qmh_rms_inv(ss - d, n, eps);
        if (inv != qmh_rms_inv(ss + d, n, eps)) {  // uniform; serial sum as the reference
            if (tid == 0) {
                double s2 = 0.0;
                for (int i = 0; i < n; i++) s2 += (double)row[i] * (double)row[i];
                red[NT / 64] = s2;
            }
            __syncthreads();
            inv = qmh_rms_inv(red[NT / 64], n, eps);
        }
    }
    // (x*inv)*w as the reference; rounds are uniform (DPP needs all 8 lanes of a block)
    if (held) {
#pragma unroll
        for (int r = 0; r < PQ_R; r++)
            if (r < R) {
                const int b = r * (NT / 8) + (tid >> 3), i4 = b * 32 + sub * 4;
                float v[4];
#pragma unroll
                for (int j = 0; j < 4; j++)
                    v[j] = w ? ((b < nb && i4 + j < n) ? xv[r][j] * inv * w[i4 + j] : 0.0f) : xv[r][j];
                pf_quant_block(v, b, nb, p, sub, xc, xd, PP, perm8);
            }
    } else {
        for (int r = 0; r < R; r++) {
            const int b = r * (NT / 8) + (tid >> 3), i4 = b * 32 + sub * 4;
            float v[4];
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const bool in = b < nb && i4 + j < n;
                v[j] = in ? (w ? row[i4 + j] * inv * w[i4 + j] : row[i4 + j]) : 0.0f;
            }
            pf_quant_block(v, b, nb, p, sub, xc, xd, PP, perm8);
        }
    }
}

// k_pf_quant for rows of n % 4 == 0 values (16-byte aligned rows and gain) in RR rounds: each
// thread's 4 values of a round are one 16-byte buffer load whose range check (n*4 bytes) zeroes
// what lies past the row, so all of a thread's loads (row and gain) issue at once, before the
// sum. The scale 1/sqrt(ss/n + eps) takes the margin test first, as the decode prologue.
typedef uint32_t pf_v4u __attribute__((ext_vector_type(4)));
template <int NT, int RR, bool NORM>
__global__ __launch_bounds__(NT) void k_pf_quant4(const float *__restrict__ x, int ldx, const float *w, float eps,
                                                      int n, int8_t *xc, float *xd, int PP, int perm8) {
    __shared__ double red[NT / 64 + 1];
    const int p = blockIdx.x, tid = threadIdx.x, nb = (n + 31) / 32, sub = tid & 7;
    const float *row = x + (size_t)p * ldx;
    const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc((void *)row, (short)0, n * 4, 0x00020000);
    pf_v4u xv[RR], wv[RR];
#pragma unroll
    for (int r = 0; r < RR; r++) xv[r] = __builtin_amdgcn_raw_buffer_load_b128(rx, (r * NT + tid) * 16, 0, 0);
    float inv = 1.0f;
    if (NORM) {
        const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc((void *)w, (short)0, n * 4, 0x00020000);
#pragma unroll
        for (int r = 0; r < RR; r++) wv[r] = __builtin_amdgcn_raw_buffer_load_b128(rw, (r * NT + tid) * 16, 0, 0);
        double ss = 0.0;  // values past the row load as +0
#pragma unroll
        for (int r = 0; r < RR; r++)
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const double v = (double)__uint_as_float(xv[r][j]);
                ss += v * v;
            }
        // wave butterflies, then the waves in order; red is not reused, so one barrier publishes
        ss = qmh_wave_sum_d(ss);
        if ((tid & 63) == 0) red[tid >> 6] = ss;
        __syncthreads();
        ss = 0.0;
#pragma unroll
        for (int k = 0; k < NT / 64; k++) ss += red[k];
        // the same ss in every thread: uniform branches
        if (!qmh_rms_inv_margin(ss, n, nb * 32, eps, &inv)) {
            const double d = qmh_sum_slack(ss, nb * 32);
            inv = qmh_rms_inv(ss - d, n, eps);
            if (inv != qmh_rms_inv(ss + d, n, eps)) {  // the reference's serial sum
                if (tid == 0) {
                    double s2 = 0.0;
                    for (int i = 0; i < n; i++) s2 += (double)row[i] * (double)row[i];
                    red[NT / 64] = s2;
                }
                __syncthreads();
                inv = qmh_rms_inv(red[NT / 64], n, eps);
            }
        }
    }
    // (x*inv)*w as the reference; rounds are uniform (DPP needs all 8 lanes of a block)
#pragma unroll
    for (int r = 0; r < RR; r++)
        if (r * (NT / 8) < nb) {
            const int b = r * (NT / 8) + (tid >> 3), i4 = b * 32 + sub * 4;
            float v[4];
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const float xe = __uint_as_float(xv[r][j]);
                v[j] = NORM ? ((b < nb && i4 + j < n) ? xe * inv * __uint_as_float(wv[r][j]) : 0.0f) : xe;
            }
            pf_quant_block(v, b, nb, p, sub, xc, xd, PP, perm8);
        }
}

template <int NT, bool NORM>
static void pf_quant4_launch(int RR, int P, hipStream_t s, const float *x, int ldx, const float *w, float eps, int n,
                             int8_t *xc, float *xd, int PP, int perm8) {
#define PQ4(R_) hipLaunchKernelGGL((k_pf_quant4<NT, R_, NORM>), dim3(P), dim3(NT), 0, s, x, ldx, w, eps, n, xc, xd, PP, perm8)
    switch (RR) {
    case 1: PQ4(1); break;
    case 2: PQ4(2); break;
    case 4: PQ4(4); break;
    case 8: PQ4(8); break;
    default: PQ4(16); break;
    }
#undef PQ4
}

extern "C" int qmh_launch_pf_quant(const float *x, int ldx, const float *w, float eps, int n, int P, int8_t *xc,
                                   float *xd, int PP, int perm8, void *stream) {
    // a few rows (batched decode): 1024 threads per row, one round of loads for a 4096-value row
    // and 16 waves to wait on them; many rows (prefill): 512 threads (256 and 1024 were 0.3-0.5%
    // slower at 512 rows)
    const int NT = P <= 16 ? 1024 : 512, nb = (n + 31) / 32, R = (nb + NT / 8 - 1) / (NT / 8);
    const bool vec = n % 4 == 0 && ldx % 4 == 0 && ((uintptr_t)x & 15) == 0 && ((uintptr_t)w & 15) == 0;
    hipStream_t s = (hipStream_t)stream;
    if (vec && R <= PQ_R) {
        const int RR = R <= 1 ? 1 : R <= 2 ? 2 : R <= 4 ? 4 : R <= 8 ? 8 : 16;
        if (NT == 1024) {
            if (w) pf_quant4_launch<1024, true>(RR, P, s, x, ldx, w, eps, n, xc, xd, PP, perm8);
            else pf_quant4_launch<1024, false>(RR, P, s, x, ldx, w, eps, n, xc, xd, PP, perm8);
        } else {
            if (w) pf_quant4_launch<512, true>(RR, P, s, x, ldx, w, eps, n, xc, xd, PP, perm8);
            else pf_quant4_launch<512, false>(RR, P, s, x, ldx, w, eps, n, xc, xd, PP, perm8);
        }
    } else if (NT == 1024) {
        hipLaunchKernelGGL(k_pf_quant<1024>, dim3(P), dim3(1024), 0, s, x, ldx, w, eps, n, xc, xd, PP, perm8);
    } else {
        hipLaunchKernelGGL(k_pf_quant<QMH_WG>, dim3(P), dim3(QMH_WG), 0, s, x, ldx, w, eps, n, xc, xd, PP, perm8);
    }
    return (int)hipGetLastError();
}

// ============================================================================ matmul
//
// One wave: NR 16-row tiles x TW 16-token tiles, all blocks in order; 4 waves per workgroup
// take consecutive 16*NR-row groups of one token group. Operands come straight from memory
// (weights once per token group, activations from L2), PD blocks ahead of the multiplies.

__device__ __forceinline__ long pf_q4_operand(uint32_t w) {
    // 8 nibbles -> 8 signed int8 (q - 8): low nibbles (e0 e2 e4 e6), then high (e1 e3 e5 e7).
    // Per byte, q + 0x78 stays below 0x100 (no carry into the next byte), and flipping its top
    // bit gives q - 8 in two's complement: 0 -> 0xf8, 8 -> 0x00, 15 -> 0x07.
    const uint32_t lo = ((w & 0x0f0f0f0fu) + 0x78787878u) ^ 0x80808080u;
    const uint32_t hi = (((w >> 4) & 0x0f0f0f0fu) + 0x78787878u) ^ 0x80808080u;
    return (long)(((uint64_t)hi << 32) | lo);
}

// slot of block 0 of a weight row: plain tiles, or interleaved (W1 | W3) tiles with tile_r/2
// rows of each matrix (half 0: W1, 1: W3); block b adds b*tile_r
__device__ __forceinline__ uint32_t pf_slot0(const qmh_pf_args &a, int row, int half) {
    if (a.il) {
        const int h = a.tile_r / 2;
        return (uint32_t)(row / h) * a.nb * a.tile_r + row % h + half * h;
    }
    return (uint32_t)(row / a.tile_r) * a.nb * a.tile_r + row % a.tile_r;
}

// NM: matrices per wave (2 for the W1 | W3 SwiGLU pair); NR: 16-row tiles per wave (each
// activation operand feeds NM*NR MFMAs); TW: 16-token tiles per wave
template <int NM, int NR, int TW>
struct PfBlock {
    long A[NM][NR];   // raw weight codes: 8 int8 (Q8_0) or 4 nibble bytes (Q4_0, low word)
    uint2 sc[NM][NR]; // the fp16 scales of the lane's 4 D rows (k_sk_gemm)
    uint32_t wh[NM][NR];  // the fp16 scale of the lane's A row (k_pf_gemm)
    long B[TW];
    float dx[TW];
};

// Per-lane byte/element offsets of the operands, fixed over the blocks: the loop adds only the
// block's uniform base, so the loads take a scalar base and these offsets. Rows past the
// allocated slots read row 0 instead: each D row depends only on its own A row, and those rows
// are never stored.
template <int NM, int NR>
struct PfLane {
    uint32_t a[NM][NR], s[NM][NR];  // weight codes (bytes), scales (elements) at block 0
    uint32_t w[NM][NR];             // k_pf_gemm: the scale (element) of the lane's A row at block 0
    uint32_t x, d;                  // activation codes (bytes), scales (elements) of token tile 0
};

// Loads only: no value is used here, so the wait for these loads falls where the block is
// multiplied, PD blocks later.
// PM: the scales as k_pf_gemm takes them (one per A row, for the scale MFMA), else the 4 of the
// lane's D rows.
template <int WT, int NM, int NR, int TW, bool PM = false>
__device__ __forceinline__ void pf_load(const qmh_pf_args &a, int b, const PfLane<NM, NR> &ln,
                                        PfBlock<NM, NR, TW> &o) {
    constexpr int CB = WT == QMH_Q8 ? 32 : 16;
    const uint8_t *cb = a.codes + (size_t)b * a.tile_r * CB;
    const uint16_t *sb = a.scales + (size_t)b * a.tile_r;
#pragma unroll
    for (int m = 0; m < NM; m++)
#pragma unroll
        for (int r = 0; r < NR; r++) {
            if (WT == QMH_Q8) o.A[m][r] = *(const long *)(cb + ln.a[m][r]);
            else o.A[m][r] = (long)*(const uint32_t *)(cb + ln.a[m][r]);
            if (PM) o.wh[m][r] = sb[ln.w[m][r]];
            else o.sc[m][r] = *(const uint2 *)(sb + ln.s[m][r]);
        }
    const int8_t *xb = a.xc + (size_t)b * a.PP * 32;
    const float *db = a.xd + (size_t)b * a.PP;
#pragma unroll
    for (int tt = 0; tt < TW; tt++) {
        o.B[tt] = *(const long *)(xb + ln.x + tt * 512);
        o.dx[tt] = db[ln.d + tt * 16];
    }
}

// one block into the chains: s = s + (float)acc * (dw * dx) per (row, token) pair. Two MFMAs per
// (row tile, token tile): the block's exact int32 dots, and the scale products dw * dx as the outer
// product of the row tile's 16 fp16 scales and the token tile's 16 (k = 0 of an f16 MFMA; every
// other k is 0 * 0). The product of two fp16 values is exact in fp32, so the MFMA returns the
// reference's dw * dx bit for bit (but +0 for -0: the chain starts at +0 and never holds -0, so
// s + (+0) == s + (-0) and the term's zero sign changes nothing); the VALU keeps the conversion,
// the multiply and the add, in the reference's order. k0 is 0xffff in the lanes of k = 0..3
// (lane / 16 == 0), else 0.
// The MFMAs of the next (row tile, token tile) pair go out, into their own registers, before the
// terms of the current one, so the multiplies run under the float work instead of each waiting for
// the previous results to be consumed. Every accumulator's chain stays in block order.
template <int WT, int NM, int NR, int TW>
__device__ __forceinline__ void pf_mul(const PfBlock<NM, NR, TW> &cur, float (&s)[NM][NR][TW][4], uint32_t k0) {
    constexpr int Q = NM * NR, U = Q * TW;  // pair u: row tile (m, r) = (q / NR, q % NR), q = u / TW; tt = u % TW
    pf_v4h Bs[TW];                          // token tile tt's scales at k = 0
#pragma unroll
    for (int tt = 0; tt < TW; tt++) {
        const uint32_t h = (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)cur.dx[tt]) & k0;  // exact: dx is fp16
        Bs[tt] = __builtin_bit_cast(pf_v4h, make_uint2(h, 0u));
    }
    long Am[Q];
    pf_v4h As[Q];  // row tile q's scales at k = 0
#pragma unroll
    for (int q = 0; q < Q; q++) {
        Am[q] = WT == QMH_Q8 ? cur.A[q / NR][q % NR] : pf_q4_operand((uint32_t)cur.A[q / NR][q % NR]);
        As[q] = __builtin_bit_cast(pf_v4h, make_uint2(cur.wh[q / NR][q % NR] & k0, 0u));
    }
    pf_v4i acc[2];
    pf_v4f pw[2];
    auto issue = [&](int u, pf_v4i &d, pf_v4f &pd) {
        const pf_v4i z = {0, 0, 0, 0};
        const pf_v4f zf = {0.0f, 0.0f, 0.0f, 0.0f};
        d = __builtin_amdgcn_mfma_i32_16x16x32_i8(Am[u / TW], cur.B[u % TW], z, 0, 0, 0);
        pd = __builtin_amdgcn_mfma_f32_16x16x16f16(As[u / TW], Bs[u % TW], zf, 0, 0, 0);
    };
    issue(0, acc[0], pw[0]);
#pragma unroll
    for (int u = 0; u < U; u++) {
        if (u + 1 < U) issue(u + 1, acc[(u + 1) & 1], pw[(u + 1) & 1]);
        const int q = u / TW, m = q / NR, r = q % NR, tt = u % TW;
#pragma unroll
        for (int e = 0; e < 4; e++) s[m][r][tt][e] = s[m][r][tt][e] + (float)acc[u & 1][e] * pw[u & 1][e];
    }
}

// one output of the matmul: y = row's value for token p (up: the W3 value of the SwiGLU pair;
// partner: the value of row ^ 1, RoPE's pair), stored as the epilogue asks
__device__ __forceinline__ void pf_store(const qmh_pf_args &a, int row, int p, float y, float up, float partner) {
    if (a.epi == QMH_PF_STORE) {
        a.out0[(size_t)p * a.ld0 + row] = y;
    } else if (a.epi == QMH_PF_ADD) {  // x += W x' (src/model.c:179,186)
        a.out0[(size_t)p * a.ld0 + row] = a.out0[(size_t)p * a.ld0 + row] + y;
    } else if (a.epi == QMH_PF_SWIGLU) {  // silu(g)*u (src/ops.c:128-133)
        a.out0[(size_t)p * a.ld0 + row] = y / (1.0f + qmh_expf(-y)) * up;
    } else {  // QKV: rope on q and k (src/ops.c:114-126), k/v into the caches
        const int pos = a.pos_arr ? a.pos_arr[p] : a.pos0 + p;
        float *kc = a.out1 + (size_t)p * a.kv_stride, *vc = a.out2 + (size_t)p * a.kv_stride;
        if (row < a.seg2) {
            const int local = row < a.seg1 ? row : row - a.seg1;
            const float *cs = a.rope + ((size_t)pos * (a.head_dim >> 1) + ((local % a.head_dim) >> 1)) * 2;
            const float c = cs[0], sn = cs[1];
            const float v = (local & 1) == 0 ? (y * c - partner * sn) : (partner * sn + y * c);
            if (row < a.seg1) a.out0[(size_t)p * a.ld0 + local] = v;
            else kc[(size_t)local * a.max_seq + pos] = v;
        } else {
            vc[(size_t)pos * a.kvd + (row - a.seg2)] = y;
        }
    }
}

template <int WT, int NM, int NR, int TW, int PD>
__global__ __launch_bounds__(QMH_WG) void k_pf_gemm(qmh_pf_args a) {
    const int wave = threadIdx.x >> 6, l = threadIdx.x & 63, kq = l >> 4;
    const int r0 = (blockIdx.y * (QMH_WG / 64) + wave) * 16 * NR;  // the wave's 16*NR rows
    const int t0 = blockIdx.x * 16 * TW;                           // the wave's first token
    if (r0 >= a.rows) return;
    constexpr int CB = WT == QMH_Q8 ? 32 : 16;
    PfLane<NM, NR> ln;
#pragma unroll
    for (int r = 0; r < NR; r++) {
        const int row = r0 + 16 * r + (l & 15);  // the lane's A row
#pragma unroll
        for (int m = 0; m < NM; m++) {
            ln.a[m][r] = pf_slot0(a, row < a.rows_alloc ? row : 0, m) * CB + (WT == QMH_Q8 ? 8 : 4) * kq;
            ln.w[m][r] = pf_slot0(a, row < a.rows_alloc ? row : 0, m);
        }
    }
    ln.x = (uint32_t)(t0 + (l & 15)) * 32 + 8 * kq;
    ln.d = (uint32_t)(t0 + (l & 15));
    const uint32_t k0 = kq == 0 ? 0xffffu : 0u;
    float s[NM][NR][TW][4];
#pragma unroll
    for (int m = 0; m < NM; m++)
#pragma unroll
        for (int r = 0; r < NR; r++)
#pragma unroll
            for (int tt = 0; tt < TW; tt++)
#pragma unroll
                for (int e = 0; e < 4; e++) s[m][r][tt][e] = 0.0f;
    // PD blocks in flight ahead of the one multiplied: a ring of PD + 1 operand sets indexed
    // statically (the group loop is unrolled PD + 1 times), so no operand is copied and each
    // wait is for loads issued PD blocks earlier. Invariant at the top of a group starting at
    // block b0: ring[j] holds block b0 + j, j < PD.
    PfBlock<NM, NR, TW> ring[PD + 1];
#pragma unroll
    for (int j = 0; j < PD; j++) pf_load<WT, NM, NR, TW, true>(a, j < a.nb ? j : a.nb - 1, ln, ring[j]);
    int b0 = 0;
    for (; b0 + PD < a.nb; b0 += PD + 1) {
#pragma unroll
        for (int j = 0; j <= PD; j++) {
            const int bn = b0 + j + PD;
            pf_load<WT, NM, NR, TW, true>(a, bn < a.nb ? bn : a.nb - 1, ln, ring[(j + PD) % (PD + 1)]);
            pf_mul<WT, NM, NR, TW>(ring[j], s, k0);
        }
    }
#pragma unroll
    for (int j = 0; j < PD; j++)
        if (b0 + j < a.nb) pf_mul<WT, NM, NR, TW>(ring[j], s, k0);
    // epilogues: lane l holds rows r0 + 16*r + 4*kq + e (e < 4) of tokens t0 + 16*tt + l%16
    if (NR == 2 && a.epi == QMH_PF_SWIGLU && a.qxc) {  // uniform
        // W2's input as its Q8_0 image: the wave's 32 rows (r0 % 32 == 0) are block r0/32 of each of
        // its tokens; lanes l, l^16, l^32, l^48 hold a token's 32 values (8 each: elements
        // 16*r + 4*kq + e). The same steps as k_pf_quant's block (src/quant.c:27-52): amax, the fp16
        // scale, the codes; rows past `rows` are 0 there and here.
        const int b = r0 >> 5;
#pragma unroll
        for (int tt = 0; tt < TW; tt++) {
            const int p = t0 + 16 * tt + (l & 15);
            float v[NR][4], m = 0.0f;
#pragma unroll
            for (int r = 0; r < NR; r++)
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const int row = r0 + 16 * r + 4 * kq + e;
                    const float y = s[0][r][tt][e], up = s[NM - 1][r][tt][e];
                    v[r][e] = row < a.rows ? y / (1.0f + qmh_expf(-y)) * up : 0.0f;  // silu(g)*u (src/ops.c:128-133)
                    const float av = fabsf(v[r][e]);
                    m = av > m ? av : m;
                }
            float o = __shfl_xor(m, 16);
            m = o > m ? o : m;
            o = __shfl_xor(m, 32);
            m = o > m ? o : m;
            const float dd = qmh_h2f(qmh_f2h(qmh_div127(m)));
            const float rinv = qmh_rcp(dd);
#pragma unroll
            for (int r = 0; r < NR; r++) {
                int q[4];
                qmh_q8_codes4(v[r], dd, rinv, q);
                const uint32_t b0 = (uint32_t)q[0] & 0xffu, b1 = (uint32_t)q[1] & 0xffu, b2 = (uint32_t)q[2] & 0xffu,
                               b3 = (uint32_t)q[3] & 0xffu;
                // bytes 16*r + 4*kq .. +3 of the block; the Q4_0 order (8g+e at 8g + {0,4,1,5,2,6,3,7}[e])
                // by a half-word swap with lane l^16, as in k_pf_quant
                const uint32_t pk = b0 | (b2 << 8) | (b1 << 16) | (b3 << 24);
                const uint32_t pp = (uint32_t)__shfl_xor((int)pk, 16);
                const uint32_t w = !a.qperm8 ? (b0 | (b1 << 8) | (b2 << 16) | (b3 << 24))
                                   : (kq & 1) == 0 ? ((pk & 0xffffu) | (pp << 16)) : ((pp >> 16) | (pk & 0xffff0000u));
                if (p < a.P) *(uint32_t *)(a.qxc + ((size_t)b * a.PP + p) * 32 + 16 * r + 4 * kq) = w;
            }
            if (p < a.P && kq == 0) a.qxd[(size_t)b * a.PP + p] = dd;
        }
        return;
    }
#pragma unroll
    for (int r = 0; r < NR; r++)
#pragma unroll
        for (int tt = 0; tt < TW; tt++) {
            const int p = t0 + 16 * tt + (l & 15);
            if (p >= a.P) continue;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const int row = r0 + 16 * r + 4 * kq + e;
                if (row >= a.rows) continue;
                // rows 2i, 2i+1 share the lane (RoPE partner)
                pf_store(a, row, p, s[0][r][tt][e], s[NM - 1][r][tt][e], s[0][r][tt][e ^ 1]);
            }
        }
}

// Skinny matmul for decode-sized batches (P <= 16*TT tokens, TT <= 4): one workgroup per 16-row group
// streams every block of its rows once for all tokens. The blocks pass in rounds of as many as
// fit the LDS budget at this P: wave w takes blocks base + 8j + w in batches of PD (each batch's
// loads all in flight, no barrier inside a round), takes each block's exact int32 dot for TT
// token tiles from MFMAs with a zero accumulator, and stores the term (float)acc*(dw*dx) in LDS
// at [matrix][block in round][token][row]; after the round one thread per (row, token) pair
// extends that pair's serial chain over the round's blocks in order (the reference's order).
// After the last round each pair runs the epilogue. Dynamic LDS: one round's terms, at most SK_LDS.
#define SK_WG 512
#define SK_LDS (128 * 1024)
// blocks per round: a multiple of 8 that fits the LDS budget at P tokens (the launch gives the
// kernel exactly NM*16*P*4 bytes per block of a round)
__host__ __device__ inline int sk_round(int nb, int nm, int P) {
    const int fit = (SK_LDS / (nm * 16 * P * 4)) & ~7, all = (nb + 7) & ~7;
    return fit < all ? fit : all;
}
template <int WT, int NM, int TT, int PD>
__global__ __launch_bounds__(SK_WG) void k_sk_gemm(qmh_pf_args a) {
    constexpr int PT = 16 * TT;
    constexpr int NPAIR = 16 * PT / SK_WG > 0 ? 16 * PT / SK_WG : 1;  // (row, token) pairs per thread
    extern __shared__ float T[];
    const int wave = threadIdx.x >> 6, l = threadIdx.x & 63, kq = l >> 4, tok = l & 15;
    const int r0 = blockIdx.x * 16, P = a.P, nb = a.nb;
    const int rblk = sk_round(nb, NM, P);
    constexpr int CB = WT == QMH_Q8 ? 32 : 16;
    PfLane<NM, 1> ln;
    {
        const int row = r0 + tok;  // the lane's A row
#pragma unroll
        for (int m = 0; m < NM; m++) {
            ln.a[m][0] = pf_slot0(a, row < a.rows_alloc ? row : 0, m) * CB + (WT == QMH_Q8 ? 8 : 4) * kq;
            ln.w[m][0] = pf_slot0(a, row < a.rows_alloc ? row : 0, m);
        }
    }
    const uint32_t kmask = kq == 0 ? 0xffffu : 0u;  // lanes of k = 0..3
    ln.x = (uint32_t)tok * 32 + 8 * kq;
    ln.d = (uint32_t)tok;
    float s[NPAIR][NM];
#pragma unroll
    for (int k = 0; k < NPAIR; k++)
#pragma unroll
        for (int m = 0; m < NM; m++) s[k][m] = 0.0f;
    for (int base = 0; base < nb; base += rblk) {
        const int nr = min(rblk, nb - base);
        for (int k0 = 0; 8 * k0 + wave < nr; k0 += PD) {  // uniform per wave
            PfBlock<NM, 1, TT> blk[PD];
#pragma unroll
            for (int j = 0; j < PD; j++) {
                const int jb = 8 * (k0 + j) + wave;
                pf_load<WT, NM, 1, TT, true>(a, base + (jb < nr ? jb : nr - 1), ln, blk[j]);
            }
#pragma unroll
            for (int j = 0; j < PD; j++) {
                const int jb = 8 * (k0 + j) + wave;
                if (jb < nr) {  // uniform per wave
                    // every MFMA of the block first, each into its own registers, then the terms:
                    // the multiplies overlap instead of each waiting for the previous results. The
                    // scale products dw * dx come from an f16 MFMA with the scales at k = 0, as in
                    // k_pf_gemm (exact: a product of two fp16 values)
                    pf_v4i acc[NM][TT];
                    pf_v4f pw[NM][TT];
                    pf_v4h Bs[TT];
#pragma unroll
                    for (int tt = 0; tt < TT; tt++) {
                        const uint32_t h = (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)blk[j].dx[tt]) & kmask;
                        Bs[tt] = __builtin_bit_cast(pf_v4h, make_uint2(h, 0u));
                    }
#pragma unroll
                    for (int m = 0; m < NM; m++) {
                        const long Am = WT == QMH_Q8 ? blk[j].A[m][0] : pf_q4_operand((uint32_t)blk[j].A[m][0]);
                        const pf_v4h As = __builtin_bit_cast(pf_v4h, make_uint2(blk[j].wh[m][0] & kmask, 0u));
#pragma unroll
                        for (int tt = 0; tt < TT; tt++) {
                            const pf_v4i z = {0, 0, 0, 0};
                            const pf_v4f zf = {0.0f, 0.0f, 0.0f, 0.0f};
                            acc[m][tt] = __builtin_amdgcn_mfma_i32_16x16x32_i8(Am, blk[j].B[tt], z, 0, 0, 0);
                            pw[m][tt] = __builtin_amdgcn_mfma_f32_16x16x16f16(As, Bs[tt], zf, 0, 0, 0);
                        }
                    }
#pragma unroll
                    for (int m = 0; m < NM; m++)
#pragma unroll
                        for (int tt = 0; tt < TT; tt++) {
                            const int p = 16 * tt + tok;
                            if (p < P) {  // rows 4*kq .. +3 of token p: one 16-byte store
                                pf_v4f t;
#pragma unroll
                                for (int e = 0; e < 4; e++) t[e] = (float)acc[m][tt][e] * pw[m][tt][e];
                                *(pf_v4f *)(T + ((m * rblk + jb) * P + p) * 16 + 4 * kq) = t;
                            }
                        }
                }
            }
        }
        __syncthreads();
#pragma unroll
        for (int k = 0; k < NPAIR; k++) {
            const int c = threadIdx.x + k * SK_WG, row = c & 15, p = c >> 4;
            if (p < P)
                for (int jb = 0; jb < nr; jb++)  // the matrices' chains side by side, each in block order
#pragma unroll
                    for (int m = 0; m < NM; m++) s[k][m] = s[k][m] + T[((m * rblk + jb) * P + p) * 16 + row];
        }
        __syncthreads();
    }
#pragma unroll
    for (int k = 0; k < NPAIR; k++) {
        const int c = threadIdx.x + k * SK_WG, row = c & 15, p = c >> 4;
        const float partner = __shfl_xor(s[k][0], 1);  // row ^ 1 of the same token: RoPE's pair
        if (p < P && r0 + row < a.rows) pf_store(a, r0 + row, p, s[k][0], s[k][NM - 1], partner);
    }
}

// ============================================================================ multi-token matvec
//
// Up to BMV_P tokens (batched decode, short prompts): the decode matvec's organisation with one
// record and one term per token. A workgroup owns a contiguous range of whole tiles (contiguous
// slots: tile-major, then block, then row in tile). Its threads stream every slot once (8 Q4_0 or 4
// Q8_0 slots per thread per register set, two sets), and for each token form the block's exact int32
// dot with sdot4 against that token's activation record in LDS, then the term (float)acc * (dw * dx)
// into LDS at [token][slot]. After the stream one lane per (row, token) walks its terms in block order
// from +0 (the reference's chain) and runs the prefill epilogue (pf_store).
//
// Records: 48 bytes per (block, token), codes in the order the weights pair with (Q8_0: element
// order; Q4_0: even elements, then odd), then d (fp32), then the code sum (Q4_0: sum (q - 8) x =
// sum q x - 8 sum x, exact). They are built either from the Q8_0 image of k_pf_quant (its perm8
// groups [e0 e2 e4 e6 e1 e3 e5 e7] give their first 4 bytes to the even half and the last 4 to the
// odd half) or, for a plain input, straight from the f32 rows (bmv_records_f32).
#define BMV_P 3
#define BMV_NT 512
#define BMV_REC 48
#define BMV_CH 4  // (row, token) pairs per thread: rows of a workgroup x tokens <= 4*BMV_NT
#define BMV_LDS (160 * 1024)
__host__ __device__ inline int bmv_ntiles(const qmh_pf_args &a) {
    return a.il ? a.rows_alloc / (a.tile_r / 2) : a.rows_alloc / a.tile_r;
}
__host__ __device__ inline int bmv_tile0(int w, int ntiles, int G) { return (int)((long long)w * ntiles / G); }

// Records straight from the f32 rows of a plain (not RMSNorm'd) input, as k_pf_quant computes them:
// item k = p*nb + b is block b of token p, 8 lanes per item with 4 values each, four rounds of
// items at a time. Q4_0 consumers get the split code order.
template <int WT>
__device__ __forceinline__ void bmv_quant_item(const qmh_pf_args &a, uint8_t *rec, int k, int nk, const float (&v)[4]) {
    const int sub = threadIdx.x & 7, P = a.P, nb = a.nb, p = k / nb, b = k - p * nb;
    float m = 0.0f;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const float av = fabsf(v[j]);
        m = av > m ? av : m;
    }
    m = qmh_amax8(m);
    const float dd = qmh_h2f(qmh_f2h(qmh_div127(m)));
    int q[4];
    qmh_q8_codes4(v, dd, qmh_rcp(dd), q);
    const int qs = qmh_sum8(q[0] + q[1] + q[2] + q[3]);
    if (k < nk) {
        uint8_t *rp = rec + (size_t)(b * P + p) * BMV_REC;
        if (WT == QMH_Q4) {  // elements 4s, 4s+2 at 2s, 2s+1; 4s+1, 4s+3 at 16+2s, 16+2s+1
            *(uint16_t *)(rp + 2 * sub) = (uint16_t)((q[0] & 0xff) | (q[2] & 0xff) << 8);
            *(uint16_t *)(rp + 16 + 2 * sub) = (uint16_t)((q[1] & 0xff) | (q[3] & 0xff) << 8);
        } else {
            *(uint32_t *)(rp + 4 * sub) =
                (uint32_t)((q[0] & 0xff) | (q[1] & 0xff) << 8 | (q[2] & 0xff) << 16 | (q[3] & 0xff) << 24);
        }
        if (sub == 0) {
            *(float *)(rp + 32) = dd;
            *(int *)(rp + 36) = qs;
        }
    }
}

template <int WT>
__device__ __forceinline__ void bmv_records_f32(const qmh_pf_args &a, uint8_t *rec) {
    const int tid = threadIdx.x, sub = tid & 7, P = a.P, nb = a.nb, n = a.nxf;
    const int nk = P * nb, NR = (nk + BMV_NT / 8 - 1) / (BMV_NT / 8);
    for (int r0 = 0; r0 < NR; r0 += 4) {  // uniform: DPP needs all 8 lanes of an item
        float xv[4][4];
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const int k = (r0 + u) * (BMV_NT / 8) + (tid >> 3), p = k / nb, i0 = (k - p * nb) * 32 + 4 * sub;
#pragma unroll
            for (int j = 0; j < 4; j++)
                xv[u][j] = (r0 + u < NR && k < nk && i0 + j < n) ? a.xf[(size_t)p * a.ldxf + i0 + j] : 0.0f;
        }
#pragma unroll
        for (int u = 0; u < 4; u++)
            if (r0 + u < NR) bmv_quant_item<WT>(a, rec, (r0 + u) * (BMV_NT / 8) + (tid >> 3), nk, xv[u]);
    }
}

// MP: the largest token count P the instance serves (its per-token loop is unrolled MP times)
template <int WT, int MP>
__global__ __launch_bounds__(BMV_NT, 4) void k_bmv(qmh_pf_args a) {  // 4 waves per SIMD: two per CU
    constexpr int CB = WT == QMH_Q8 ? 32 : 16;  // code bytes per slot
    constexpr int NV = CB / 16;
    constexpr int U = WT == QMH_Q8 ? 4 : 8;      // slots per thread per register set
    extern __shared__ __align__(16) uint8_t smem[];
    const int tid = threadIdx.x, P = a.P, nb = a.nb, R = a.tile_r, lgR = __builtin_ctz((unsigned)R);
    const int ntiles = bmv_ntiles(a);
    const int t0 = bmv_tile0(blockIdx.x, ntiles, gridDim.x), t1 = bmv_tile0(blockIdx.x + 1, ntiles, gridDim.x);
    const int ntw = t1 - t0;
    if (ntw <= 0) return;  // the host launches at most ntiles workgroups
    // blocks per LDS round: all of them, or (one tile per workgroup) as many as let two workgroups
    // share a CU; each round's terms extend the chains before the next round overwrites them
    const int bq = a.bmv_bq > 0 && a.bmv_bq < nb && ntw == 1 ? a.bmv_bq : nb;
    float *T = (float *)(smem + (size_t)nb * P * BMV_REC);
    const uint8_t *cbase = a.codes + (size_t)t0 * nb * R * CB;
    const uint16_t *sbase = a.scales + (size_t)t0 * nb * R;
    uint4 cA[U][NV], cB[U][NV];
    uint32_t sA[U], sB[U];
    int q0 = 0, nbq = bq, TS = ntw * bq * R;  // the round's first block, blocks, slots
    // slot l = j*BMV_NT + tid of the round: block column (l >> lgR) = (tid >> lgR) + j*(BMV_NT >> lgR);
    // its block index in the round is that mod nbq, kept incrementally (step < nbq). With several
    // tiles there is one round (q0 = 0); with rounds there is one tile, so slot q0*R + l of the range
    auto load = [&](uint4 (&c)[U][NV], uint32_t (&sc)[U], int j0) {
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int l0 = (j0 + u) * BMV_NT + tid, l = (l0 < TS ? l0 : TS - 1) + q0 * R;
#pragma unroll
            for (int v = 0; v < NV; v++) c[u][v] = *(const uint4 *)(cbase + (size_t)l * CB + 16 * v);
            sc[u] = sbase[l];
        }
    };
    load(cA, sA, 0);

    if (a.xf) {
        bmv_records_f32<WT>(a, smem);
    } else {
    // records from the quantized image
    const int nitems = nb * P * 4;  // (block, token, 8-byte group); groups of one record in adjacent lanes
    for (int i0 = 0; i0 < nitems; i0 += BMV_NT) {
        const int it = i0 + tid, g = it & 3, bp = it >> 2, b = bp / P, p = bp - b * P;
        const bool ok = it < nitems;
        int2 v = make_int2(0, 0);
        if (ok) v = *(const int2 *)(a.xc + ((size_t)b * a.PP + p) * 32 + 8 * g);
        int sum = __builtin_amdgcn_sdot4(v.x, 0x01010101, 0, false);
        sum = __builtin_amdgcn_sdot4(v.y, 0x01010101, sum, false);
        sum += __shfl_xor(sum, 1);
        sum += __shfl_xor(sum, 2);
        if (ok) {
            uint8_t *rec = smem + (size_t)bp * BMV_REC;
            if (WT == QMH_Q4) {
                *(int *)(rec + 4 * g) = v.x;
                *(int *)(rec + 16 + 4 * g) = v.y;
            } else {
                *(int2 *)(rec + 8 * g) = v;
            }
            if (g == 0) {
                *(float *)(rec + 32) = a.xd[(size_t)b * a.PP + p];
                *(int *)(rec + 36) = sum;
            }
        }
    }
    }
    __syncthreads();

    // the rounds: stream (terms to LDS), then every chain extended over the round's blocks in order
    const int rows_w = ntw * R, npair = rows_w * P;  // pair c = p*rows_w + i: row i of the range, token p
    float yk[BMV_CH];
#pragma unroll
    for (int kc = 0; kc < BMV_CH; kc++) yk[kc] = 0.0f;
    for (q0 = 0; q0 < nb; q0 += bq) {
        nbq = nb - q0 < bq ? nb - q0 : bq;
        TS = ntw * nbq * R;
        const int nper = (TS + BMV_NT - 1) / BMV_NT, bstep = (BMV_NT >> lgR) % nbq;
        int bcur = (tid >> lgR) % nbq;
        auto compute = [&](const uint4 (&c)[U][NV], const uint32_t (&sc)[U], int j0) {
#pragma unroll
            for (int u = 0; u < U; u++) {
                const int l = (j0 + u) * BMV_NT + tid;
                if (j0 + u < nper) {  // uniform
                    const float dw = qmh_h2f((uint16_t)sc[u]);
#pragma unroll
                    for (int p = 0; p < MP; p++)
                        if (p < P) {
                            const uint8_t *rp = smem + (size_t)((q0 + bcur) * P + p) * BMV_REC;
                            const int4 x0 = *(const int4 *)rp, x1 = *(const int4 *)(rp + 16);
                            const float2 ds = *(const float2 *)(rp + 32);
                            int acc;
                            if (WT == QMH_Q4) {
                                const uint4 w = c[u][0];
                                acc = -8 * __float_as_int(ds.y);
                                acc = __builtin_amdgcn_sdot4((int)(w.x & 0x0f0f0f0fu), x0.x, acc, false);
                                acc = __builtin_amdgcn_sdot4((int)((w.x >> 4) & 0x0f0f0f0fu), x1.x, acc, false);
                                acc = __builtin_amdgcn_sdot4((int)(w.y & 0x0f0f0f0fu), x0.y, acc, false);
                                acc = __builtin_amdgcn_sdot4((int)((w.y >> 4) & 0x0f0f0f0fu), x1.y, acc, false);
                                acc = __builtin_amdgcn_sdot4((int)(w.z & 0x0f0f0f0fu), x0.z, acc, false);
                                acc = __builtin_amdgcn_sdot4((int)((w.z >> 4) & 0x0f0f0f0fu), x1.z, acc, false);
                                acc = __builtin_amdgcn_sdot4((int)(w.w & 0x0f0f0f0fu), x0.w, acc, false);
                                acc = __builtin_amdgcn_sdot4((int)((w.w >> 4) & 0x0f0f0f0fu), x1.w, acc, false);
                            } else {
                                const uint4 w0 = c[u][0], w1 = c[u][NV - 1];
                                acc = __builtin_amdgcn_sdot4((int)w0.x, x0.x, 0, false);
                                acc = __builtin_amdgcn_sdot4((int)w0.y, x0.y, acc, false);
                                acc = __builtin_amdgcn_sdot4((int)w0.z, x0.z, acc, false);
                                acc = __builtin_amdgcn_sdot4((int)w0.w, x0.w, acc, false);
                                acc = __builtin_amdgcn_sdot4((int)w1.x, x1.x, acc, false);
                                acc = __builtin_amdgcn_sdot4((int)w1.y, x1.y, acc, false);
                                acc = __builtin_amdgcn_sdot4((int)w1.z, x1.z, acc, false);
                                acc = __builtin_amdgcn_sdot4((int)w1.w, x1.w, acc, false);
                            }
                            if (l < TS) T[(size_t)p * TS + l] = (float)acc * (dw * ds.x);
                        }
                }
                bcur += bstep;
                bcur -= bcur >= nbq ? nbq : 0;
            }
        };
        if (q0 > 0) load(cA, sA, 0);  // the first round's set was issued before the records
        for (int j0 = 0; j0 < nper; j0 += 2 * U) {
            if (j0 + U < nper) load(cB, sB, j0 + U);
            compute(cA, sA, j0);
            if (j0 + 2 * U < nper) load(cA, sA, j0 + 2 * U);
            if (j0 + U < nper) compute(cB, sB, j0 + U);
        }
        __syncthreads();
#pragma unroll
        for (int kc = 0; kc < BMV_CH; kc++) {
            const int c = kc * BMV_NT + tid, p = c / rows_w, i = c - p * rows_w, tl = i >> lgR, r = i & (R - 1);
            if (c < npair) {
                const float *tp = T + (size_t)p * TS + (size_t)tl * nbq * R + r;
                float y = yk[kc];
                int b = 0;
                for (; b + 16 <= nbq; b += 16) {
                    float v[16];
#pragma unroll
                    for (int k = 0; k < 16; k++) v[k] = tp[(b + k) * R];
#pragma unroll
                    for (int k = 0; k < 16; k++) y = y + v[k];
                }
                for (; b < nbq; b++) y = y + tp[b * R];
                yk[kc] = y;
            }
        }
        __syncthreads();  // the next round's terms overwrite these
    }

    // epilogues: a tile's rows are consecutive lanes of one wave (R divides 64, rows_w is a multiple of R)
#pragma unroll
    for (int kc = 0; kc < BMV_CH; kc++)
        if (kc * BMV_NT < npair) {  // uniform
            const int c = kc * BMV_NT + tid, p = c / rows_w, i = c - p * rows_w, tl = i >> lgR, r = i & (R - 1);
            const float y = yk[kc];
            const int tile = t0 + tl;
            if (a.il) {  // rows r < R/2 of a tile are W1 rows, r + R/2 their W3 rows
                const float up = __shfl_down(y, R >> 1);
                const int row = tile * (R >> 1) + r;
                if (c < npair && r < (R >> 1) && row < a.rows) pf_store(a, row, p, y, up, 0.0f);
            } else {
                const float partner = __shfl_xor(y, 1);  // row ^ 1: RoPE's pair
                const int row = tile * R + r;
                if (c < npair && row < a.rows) pf_store(a, row, p, y, y, partner);
            }
        }
}

// Wave shape of the matmuls (timed on MI355X at P = 512 over the 7B shapes): 2 row tiles x 4
// token tiles per wave, 2 blocks loaded ahead. Fewer tiles per wave issue more loads per MFMA;
// more leave too few waves to cover the latency at P = 512. W1 | W3 loads 1 block ahead: that
// holds it to 166 VGPRs, three waves per SIMD, so its 2752 wave tiles at P = 512 (7B shapes) run
// in one round of 3072 slots instead of 1.34 rounds of 2048 (20.45 -> 20.02 ms per 512-token
// prefill); the other matrices lose at depth 1 (23.5 ms with every one there).
enum { PF_NR = 2, PF_TW = 4, PF_PD = 2, PF_PD13 = 1 };

extern "C" int qmh_launch_pf_gemm(const qmh_pf_args *a, void *stream) {
    if (a->PP % 128 || a->P > a->PP || a->P < 1 || a->nb < 1) return (int)hipErrorInvalidValue;
    if ((a->epi == QMH_PF_SWIGLU) != (a->il != 0)) return (int)hipErrorInvalidValue;
    if (a->dtype != QMH_Q4 && a->dtype != QMH_Q8) return (int)hipErrorInvalidValue;
    // the image output exists only in the tiled matmul's SwiGLU epilogue (more than QMH_PF_SKINNY_P tokens)
    if (a->qxc && (a->epi != QMH_PF_SWIGLU || !a->qxd || a->P <= QMH_PF_SKINNY_P || PF_NR != 2)) return (int)hipErrorInvalidValue;
    hipStream_t s = (hipStream_t)stream;
    if (a->xf && (a->nxf < 1 || a->nxf > 32 * a->nb || a->ldxf < a->nxf)) return (int)hipErrorInvalidValue;
    // the multi-token matvec when one tile's terms fit its LDS with the records. It quantizes a plain
    // input (Wo's, W2's) itself: timed on MI355X at 1-4 tokens, that saves 5-9 us per matmul over
    // k_pf_quant's launch, while an RMSNorm'd input quantized in every workgroup was 6 us slower.
    const int ntiles = bmv_ntiles(*a);
    const size_t rec = (size_t)a->nb * a->P * BMV_REC, per_tile = (size_t)a->P * a->tile_r * a->nb * sizeof(float);
    const bool bmv = a->P <= BMV_P && rec + per_tile <= BMV_LDS &&
                     (size_t)a->tile_r * a->P * ((ntiles + 255) / 256) <= (size_t)BMV_CH * BMV_NT;
    const bool fuse = bmv && a->xf && !a->norm_w;
    if (a->xf && !fuse) {  // the quantized image first
        const int rc = qmh_launch_pf_quant(a->xf, a->ldxf, a->norm_w, a->eps, a->nxf, a->P, (int8_t *)a->xc,
                                           (float *)a->xd, a->PP, a->dtype == QMH_Q4, stream);
        if (rc) return rc;
    }
    if (bmv) {
        qmh_pf_args b = *a;
        if (!fuse) b.xf = nullptr;
        // whole tiles per workgroup: about one workgroup per CU (256), fewer tiles if LDS asks
        const int fit = (int)((BMV_LDS - rec) / per_tile), want = ntiles / 256 > 1 ? ntiles / 256 : 1;
        const int k = want < fit ? want : fit, G = (ntiles + k - 1) / k;
        size_t lds = rec + (size_t)((ntiles + G - 1) / G) * per_tile;
        // one tile per workgroup, more workgroups than CUs and room for one per CU: LDS rounds of bq
        // blocks so that two share a CU
        b.bmv_bq = 0;
        const size_t per_block = (size_t)a->P * a->tile_r * sizeof(float);
        if (k == 1 && ntiles > 256 && 2 * lds > BMV_LDS && 2 * rec < BMV_LDS) {
            const int bq = (int)((BMV_LDS / 2 - rec) / per_block);
            if (bq >= 16 && bq < a->nb) {
                b.bmv_bq = bq;
                lds = rec + (size_t)bq * per_block;
            }
        }
#define BMV_GO(MP_)                                                                                    \
    do {                                                                                                 \
        if (a->dtype == QMH_Q4) hipLaunchKernelGGL((k_bmv<QMH_Q4, MP_>), dim3(G), dim3(BMV_NT), lds, s, b); \
        else hipLaunchKernelGGL((k_bmv<QMH_Q8, MP_>), dim3(G), dim3(BMV_NT), lds, s, b);                  \
    } while (0)
        // one instance for 1-2 tokens, one for 3 (the single-token instance was 2% slower at one
        // sequence than the 2-token one)
        static_assert(BMV_P == 3, "k_bmv instances for up to 3 tokens");
        if (a->P <= 2) BMV_GO(2);
        else BMV_GO(3);
#undef BMV_GO
        return (int)hipGetLastError();
    }
    if (a->P <= QMH_PF_SKINNY_P) {  // decode-sized batches: the skinny matmul streams every weight once
        const dim3 g((a->rows + 15) / 16);
        const int nm = a->il ? 2 : 1;
        const size_t lds = (size_t)sk_round(a->nb, nm, a->P) * nm * 16 * a->P * sizeof(float);
#define SK_LAUNCH(NMV, TTV, PDV)                                                                              \
    do {                                                                                                      \
        if (a->dtype == QMH_Q4)                                                                               \
            hipLaunchKernelGGL((k_sk_gemm<QMH_Q4, NMV, TTV, PDV>), g, dim3(SK_WG), lds, s, *a);               \
        else                                                                                                  \
            hipLaunchKernelGGL((k_sk_gemm<QMH_Q8, NMV, TTV, PDV>), g, dim3(SK_WG), lds, s, *a);               \
    } while (0)
        // load depths timed on MI355X over the 7B shapes: for W1 | W3 up to 4 tokens, 3 blocks
        // ahead (113 VGPRs: two workgroups per CU) beat 8 by 5%; from 5 tokens 8 is ahead
        if (a->P <= 4 && a->il) {
            SK_LAUNCH(2, 1, 3);
        } else if (a->P <= 16) {
            if (a->il) SK_LAUNCH(2, 1, 8);
            else SK_LAUNCH(1, 1, 6);
        } else if (a->P <= 32) {
            if (a->il) SK_LAUNCH(2, 2, 4);
            else SK_LAUNCH(1, 2, 8);
        } else {  // 33..64 tokens: a round holds 16 (W1 | W3) or 32 blocks, 2 or 4 per wave; 2 ahead
            if (a->il) SK_LAUNCH(2, 4, 2);
            else SK_LAUNCH(1, 4, 2);
        }
#undef SK_LAUNCH
        return (int)hipGetLastError();
    }
    // token groups past P are not launched; 16 * PF_TW divides PP, so every B load stays in the
    // PP-token activation buffer
    const dim3 g((a->P + 16 * PF_TW - 1) / (16 * PF_TW), (a->rows + 64 * PF_NR - 1) / (64 * PF_NR));
    if (a->il) {
        if (a->dtype == QMH_Q4) hipLaunchKernelGGL((k_pf_gemm<QMH_Q4, 2, PF_NR, PF_TW, PF_PD13>), g, dim3(QMH_WG), 0, s, *a);
        else hipLaunchKernelGGL((k_pf_gemm<QMH_Q8, 2, PF_NR, PF_TW, PF_PD13>), g, dim3(QMH_WG), 0, s, *a);
    } else {
        if (a->dtype == QMH_Q4) hipLaunchKernelGGL((k_pf_gemm<QMH_Q4, 1, PF_NR, PF_TW, PF_PD>), g, dim3(QMH_WG), 0, s, *a);
        else hipLaunchKernelGGL((k_pf_gemm<QMH_Q8, 1, PF_NR, PF_TW, PF_PD>), g, dim3(QMH_WG), 0, s, *a);
    }
    return (int)hipGetLastError();
}

// ============================================================================ attention
//
// Scores of 16 tokens against 256 positions per workgroup (lane = position; 16 serial dot
// chains over head_dim per lane, K^T read once for the 16 tokens), each times the scale as
// src/model.c:146. Rows of att: (head, token) with max_seq entries; entries past the token's
// position are not written.
#define QMH_PF_TOK 16
__global__ __launch_bounds__(QMH_WG) void k_pf_scores(const float *__restrict__ Q, const float *__restrict__ Kt,
                                                      float *att, int P, int pos0, int n_heads, int n_kv, int hd,
                                                      int max_seq, float scale) {
    const int h = blockIdx.x, g = blockIdx.y, t = blockIdx.z * QMH_WG + threadIdx.x;
    const int p0 = g * QMH_PF_TOK, np = min(QMH_PF_TOK, P - p0);
    // a wave whose 64 positions are all past the group's last token has nothing to store (the
    // kernel has no barrier, so waves leave independently)
    if ((int)(blockIdx.z * QMH_WG + (threadIdx.x & ~63u)) > pos0 + p0 + np - 1) return;
    const int kvh = h / (n_heads / n_kv), D = n_heads * hd;
    // the group's queries, read with uniform (scalar) loads: every lane needs the same values.
    // Tokens past P read the last token's row (their scores are never stored).
    const float *qg = Q + (size_t)h * hd;
    const int tc = t < max_seq ? t : max_seq - 1;
    const float *kc = Kt + (size_t)kvh * hd * max_seq + tc;
    float s[QMH_PF_TOK];
#pragma unroll
    for (int k = 0; k < QMH_PF_TOK; k++) s[k] = 0.0f;
    // 64 K values of the lane's position in flight, then four dimensions per step (hd is a
    // multiple of 4)
    for (int d0 = 0; d0 < hd; d0 += 64) {
        float kv[64];
#pragma unroll
        for (int j = 0; j < 64; j++) kv[j] = kc[(size_t)(d0 + j < hd ? d0 + j : hd - 1) * max_seq];
#pragma unroll
        for (int j = 0; j < 64; j += 4)
            if (d0 + j < hd) {
#pragma unroll
                for (int k = 0; k < QMH_PF_TOK; k++) {
                    const float *qk = qg + (size_t)(p0 + k < P ? p0 + k : P - 1) * D + d0 + j;
                    const float4 q4 = make_float4(qk[0], qk[1], qk[2], qk[3]);
                    s[k] = s[k] + q4.x * kv[j];
                    s[k] = s[k] + q4.y * kv[j + 1];
                    s[k] = s[k] + q4.z * kv[j + 2];
                    s[k] = s[k] + q4.w * kv[j + 3];
                }
            }
    }
#pragma unroll
    for (int k = 0; k < QMH_PF_TOK; k++)
        if (k < np && t <= pos0 + p0 + k) att[((size_t)h * P + p0 + k) * max_seq + t] = s[k] * scale;
}

// The same scores blocked in registers: a workgroup takes 64 tokens x 64 positions, each thread
// 4 tokens x 4 positions (16 chains). The query and K^T tiles ([HD][64] each) are staged in LDS;
// per dimension a thread reads 4 query and 4 key values (two 16-byte LDS reads) for 32 VALU
// operations. (One token x 16 positions per lane needs 16 LDS values per 32 operations, which
// saturates the LDS return path before the VALU.) Same chains: s = +0, s = s + q[d] * k[d] over d
// in order, then s * scale.
template <int HD>
__global__ __launch_bounds__(QMH_WG) void k_pf_scores_rb(const float *__restrict__ Q, const float *__restrict__ Kt,
                                                         float *att, int P, int pos0, int n_heads, int n_kv,
                                                         int max_seq, float scale) {
    // the dimensions pass in phases of DP: 32 KB of LDS per workgroup, so that five share a CU and
    // the causal half of the tiles (1152 of 2048 at 512 tokens) runs in one round
    constexpr int DP = HD < 64 ? HD : 64;
    __shared__ __align__(16) float qs[DP * 64];  // [d][token]
    __shared__ __align__(16) float ks[DP * 64];  // [d][position]
    const int h = blockIdx.x, tid = threadIdx.x;
    const int p0 = blockIdx.y * 64, c0 = blockIdx.z * 64;
    if (c0 > pos0 + min(p0 + 63, P - 1)) return;  // the whole tile is past every token (uniform)
    const int kvh = h / (n_heads / n_kv);
    const int tg = tid >> 4, pg = tid & 15;  // tokens 4*tg .. +3, positions 4*pg .. +3
    float s[4][4];
#pragma unroll
    for (int a = 0; a < 4; a++)
#pragma unroll
        for (int b = 0; b < 4; b++) s[a][b] = 0.0f;
#pragma unroll
    for (int d0 = 0; d0 < HD; d0 += DP) {
        if (d0) __syncthreads();  // the previous phase's reads are done
        const float *kt = Kt + ((size_t)kvh * HD + d0) * max_seq;
#pragma unroll
        for (int k = 0; k < DP * 64 / QMH_WG; k++) {  // K^T rows, coalesced; positions past max_seq read the last
            const int e = k * QMH_WG + tid, t = c0 + (e & 63);
            ks[e] = kt[(size_t)(e >> 6) * max_seq + (t < max_seq ? t : max_seq - 1)];
        }
        const float *qh = Q + (size_t)h * HD + d0;
#pragma unroll
        for (int k = 0; k < DP * 64 / 4 / QMH_WG; k++) {  // 4 dimensions of one token per thread; tokens past P read the last
            const int e = k * QMH_WG + tid, tok = e & 63, d4 = e >> 6;
            const int p = p0 + tok < P ? p0 + tok : P - 1;
            const float4 v = *(const float4 *)(qh + (size_t)p * n_heads * HD + 4 * d4);
            qs[(4 * d4) * 64 + tok] = v.x;
            qs[(4 * d4 + 1) * 64 + tok] = v.y;
            qs[(4 * d4 + 2) * 64 + tok] = v.z;
            qs[(4 * d4 + 3) * 64 + tok] = v.w;
        }
        __syncthreads();
        // dimension d + KA's values are read while dimension d is used. An empty asm per step pins
        // the chains and the reads to their step: otherwise the compiler hoists every read to the
        // top and sinks the arithmetic (DP*8 live registers)
        constexpr int KA = 2;
        float4 qv[KA + 1], kv[KA + 1];
#pragma unroll
        for (int d = 0; d < KA; d++) {
            qv[d] = *(const float4 *)(qs + d * 64 + 4 * tg);
            kv[d] = *(const float4 *)(ks + d * 64 + 4 * pg);
        }
#pragma unroll
        for (int d = 0; d < DP; d++) {
            if (d + KA < DP) {
                qv[(d + KA) % (KA + 1)] = *(const float4 *)(qs + (d + KA) * 64 + 4 * tg);
                kv[(d + KA) % (KA + 1)] = *(const float4 *)(ks + (d + KA) * 64 + 4 * pg);
            }
            const float4 a4 = qv[d % (KA + 1)], b4 = kv[d % (KA + 1)];
            const float qa[4] = {a4.x, a4.y, a4.z, a4.w}, kb[4] = {b4.x, b4.y, b4.z, b4.w};
#pragma unroll
            for (int a = 0; a < 4; a++)
#pragma unroll
                for (int b = 0; b < 4; b++) s[a][b] = s[a][b] + qa[a] * kb[b];
            asm volatile("" : "+v"(s[0][0]), "+v"(s[0][1]), "+v"(s[0][2]), "+v"(s[0][3]), "+v"(s[1][0]), "+v"(s[1][1]),
                         "+v"(s[1][2]), "+v"(s[1][3]), "+v"(s[2][0]), "+v"(s[2][1]), "+v"(s[2][2]), "+v"(s[2][3]),
                         "+v"(s[3][0]), "+v"(s[3][1]), "+v"(s[3][2]), "+v"(s[3][3])::"memory");
        }
    }
#pragma unroll
    for (int a = 0; a < 4; a++) {
        const int p = p0 + 4 * tg + a;
        if (p >= P) continue;
        float *row = att + ((size_t)h * P + p) * max_seq;
#pragma unroll
        for (int b = 0; b < 4; b++) {
            const int t = c0 + 4 * pg + b;
            if (t <= pos0 + p) row[t] = s[a][b] * scale;
        }
    }
}

// softmax of one (head, token) row in place (src/ops.c:100-112), one wave per row (4 rows per
// workgroup): the max and the double sum of the exponentials by shuffles, no barrier. The final
// pass recomputes each exponential instead of storing and re-reading it (the same bits), so the
// serial fallback of the sum works from the untouched scores.
__global__ __launch_bounds__(QMH_WG) void k_pf_softmax(float *att, int P, int pos0, int max_seq) {
    const int h = blockIdx.x, p = blockIdx.y * (QMH_WG / 64) + (int)(threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (p >= P) return;  // the whole wave
    const int n = pos0 + p + 1;
    float *x = att + ((size_t)h * P + p) * max_seq;
    const float x0 = x[0];
    float m = -__builtin_inff();
    for (int t = lane; t < n; t += 64) m = x[t] > m ? x[t] : m;
    m = qmh_wave_max(m);
    if (x0 != x0) m = x0;  // the reference's scan starts from x[0]: a NaN there stays
    double sum = 0.0;
    for (int t = lane; t < n; t += 64) sum += (double)qmh_expf(x[t] - m);
    sum = qmh_wave_sum_d(sum);
    const double d = qmh_sum_slack(sum, n);
    float inv = qmh_recip_of_sum(sum - d);
    if (inv != qmh_recip_of_sum(sum + d)) {  // uniform; serial sum as the reference
        double ser = 0.0;
        if (lane == 0)
            for (int t = 0; t < n; t++) ser += (double)qmh_expf(x[t] - m);
        inv = qmh_recip_of_sum(__shfl(ser, 0));
    }
    for (int t = lane; t < n; t += 64) x[t] = qmh_expf(x[t] - m) * inv;
}

// k_pf_softmax with the row in registers (rows of up to 64*R positions): one range-checked load
// per value, all issued at once; each exponential is computed once and kept for both the sum and
// the probability (the same values k_pf_softmax computes twice). The serial fallback reads the
// scores, which stay untouched until the final stores.
template <int R>
__global__ __launch_bounds__(QMH_WG) void k_pf_softmax_r(float *att, int P, int pos0, int max_seq) {
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));  // uniform: a scalar resource
    const int h = blockIdx.x, p = blockIdx.y * (QMH_WG / 64) + wave, lane = threadIdx.x & 63;
    if (p >= P) return;  // the whole wave
    const int n = pos0 + p + 1;
    float *x = att + ((size_t)h * P + p) * max_seq;
    const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc((void *)x, (short)0, n * 4, 0x00020000);
    float xv[R];
#pragma unroll
    for (int r = 0; r < R; r++) xv[r] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rx, (r * 64 + lane) * 4, 0, 0));
    float m = -__builtin_inff();
#pragma unroll
    for (int r = 0; r < R; r++)
        if (r * 64 + lane < n) m = xv[r] > m ? xv[r] : m;
    m = qmh_wave_max(m);
    const float x0 = __shfl(xv[0], 0);
    if (x0 != x0) m = x0;  // the reference's scan starts from x[0]: a NaN there stays
    float e[R];
    double sum = 0.0;
#pragma unroll
    for (int r = 0; r < R; r++) {
        e[r] = 0.0f;
        if (r * 64 < n) {  // uniform: rounds past the row cost nothing (rows are 1 .. 64*R long)
            e[r] = qmh_expf(xv[r] - m);
            if (r * 64 + lane < n) sum += (double)e[r];
        }
    }
    sum = qmh_wave_sum_d(sum);
    const double d = qmh_sum_slack(sum, n);
    float inv = qmh_recip_of_sum(sum - d);
    if (inv != qmh_recip_of_sum(sum + d)) {  // uniform; serial sum as the reference
        double ser = 0.0;
        if (lane == 0)
            for (int t = 0; t < n; t++) ser += (double)qmh_expf(x[t] - m);
        inv = qmh_recip_of_sum(__shfl(ser, 0));
    }
#pragma unroll
    for (int r = 0; r < R; r++)
        if (r * 64 + lane < n) x[r * 64 + lane] = e[r] * inv;
}

// out[token][h*hd + i] = +0 + p_0 v_0[i] + p_1 v_1[i] + ... in position order (src/model.c:147-154);
// one workgroup per (head, 16 tokens), head_dim <= 128. V and the probabilities pass through LDS
// in chunks of 64 positions (cooperative float4 loads, the next chunk's held in registers while
// the current one is used); thread (i, half) runs column i's chains of tokens 8*half .. +7.
// The probabilities sit in LDS as [position][token], so a thread's 8 per position are two
// 16-byte reads. Positions up to pos0 + p0 are seen by every token of the group and run four at a
// time with no mask; the last 15 positions of the group (its causal diagonal) extend only the
// chains of the tokens that see them (a select, never an added zero: that would turn -0 into +0
// and propagate a NaN from V).
#define QMH_PF_VC 64
__global__ __launch_bounds__(QMH_WG) void k_pf_pv(const float *__restrict__ att, const float *__restrict__ V,
                                                  float *out, int P, int pos0, int n_heads, int n_kv, int hd,
                                                  int max_seq) {
    __shared__ __align__(16) float ps[QMH_PF_VC * QMH_PF_TOK];  // [t][token]
    __shared__ __align__(16) float vs[QMH_PF_VC * 128];         // [t][column]
    const int h = blockIdx.x, p0 = blockIdx.y * QMH_PF_TOK, np = min(QMH_PF_TOK, P - p0);
    const int kvh = h / (n_heads / n_kv), kvd = hd * n_kv, tid = threadIdx.x;
    const int tmax = pos0 + p0 + np;  // positions 0 .. tmax-1 are used by some token
    const int tall = pos0 + p0 + 1;   // positions 0 .. tall-1 are used by every token of the group
    const float *vbase = V + (size_t)kvh * hd;
    const int hd4 = hd >> 2;
    constexpr int VR = QMH_PF_VC * 128 / 4 / QMH_WG;     // float4 of V per thread per chunk
    constexpr int PR = QMH_PF_TOK * QMH_PF_VC / QMH_WG;  // probabilities per thread per chunk
    float4 vr[VR];
    float pr[PR];
    auto load = [&](int c0) {
#pragma unroll
        for (int k = 0; k < VR; k++) {
            const int e = k * QMH_WG + tid, t = e >> 5, c4 = e & 31;  // 32 float4 slots per row
            const int tc = c0 + t < tmax ? c0 + t : tmax - 1;
            vr[k] = c4 < hd4 ? *(const float4 *)(vbase + (size_t)tc * kvd + 4 * c4) : make_float4(0.f, 0.f, 0.f, 0.f);
        }
#pragma unroll
        for (int k = 0; k < PR; k++) {
            const int e = k * QMH_WG + tid, kk = e / QMH_PF_VC, t = c0 + e % QMH_PF_VC;
            pr[k] = (kk < np && t <= pos0 + p0 + kk) ? att[((size_t)h * P + p0 + kk) * max_seq + t] : 0.0f;
        }
    };
    const int i = tid & 127, half = tid >> 7;
    float acc[8];
#pragma unroll
    for (int k = 0; k < 8; k++) acc[k] = 0.0f;
    load(0);
    for (int c0 = 0; c0 < tmax; c0 += QMH_PF_VC) {
        __syncthreads();
#pragma unroll
        for (int k = 0; k < VR; k++) {
            const int e = k * QMH_WG + tid;
            *(float4 *)(vs + (e >> 5) * 128 + 4 * (e & 31)) = vr[k];
        }
#pragma unroll
        for (int k = 0; k < PR; k++) {
            const int e = k * QMH_WG + tid;
            ps[(e % QMH_PF_VC) * QMH_PF_TOK + e / QMH_PF_VC] = pr[k];
        }
        if (c0 + QMH_PF_VC < tmax) load(c0 + QMH_PF_VC);
        __syncthreads();
        if (i < hd) {
            const int nt = min(QMH_PF_VC, tmax - c0);
            const int nall = min(nt, max(tall - c0, 0));  // positions of this chunk every token sees
            const float *pp = ps + 8 * half;
            int t = 0;
            for (; t + 4 <= nall; t += 4) {
                float v[4];
                float4 pa[4], pb[4];
#pragma unroll
                for (int u = 0; u < 4; u++) {
                    v[u] = vs[(t + u) * 128 + i];
                    pa[u] = *(const float4 *)(pp + (t + u) * QMH_PF_TOK);
                    pb[u] = *(const float4 *)(pp + (t + u) * QMH_PF_TOK + 4);
                }
#pragma unroll
                for (int u = 0; u < 4; u++) {
                    acc[0] = acc[0] + pa[u].x * v[u];
                    acc[1] = acc[1] + pa[u].y * v[u];
                    acc[2] = acc[2] + pa[u].z * v[u];
                    acc[3] = acc[3] + pa[u].w * v[u];
                    acc[4] = acc[4] + pb[u].x * v[u];
                    acc[5] = acc[5] + pb[u].y * v[u];
                    acc[6] = acc[6] + pb[u].z * v[u];
                    acc[7] = acc[7] + pb[u].w * v[u];
                }
            }
            for (; t < nt; t++) {
                const float v = vs[t * 128 + i];
                const float4 pa = *(const float4 *)(pp + t * QMH_PF_TOK), pb = *(const float4 *)(pp + t * QMH_PF_TOK + 4);
                const float pk[8] = {pa.x, pa.y, pa.z, pa.w, pb.x, pb.y, pb.z, pb.w};
                const int kmin = c0 + t - (pos0 + p0);  // tokens kk >= kmin see position c0 + t
#pragma unroll
                for (int k = 0; k < 8; k++) {
                    const float nx = acc[k] + pk[k] * v;
                    acc[k] = 8 * half + k >= kmin ? nx : acc[k];
                }
            }
        }
    }
    if (i < hd)
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const int kk = 8 * half + k;
            if (kk < np) out[(size_t)(p0 + kk) * n_heads * hd + h * hd + i] = acc[k];
        }
}

// The same P·V blocked in registers for head_dim 128 and 64: each thread extends 4 tokens x 2
// columns (8 chains), a workgroup 2048/HD tokens. Per position a thread reads the 4 tokens'
// probabilities (one 16-byte LDS read) and 2 V values (8 bytes) for 16 VALU operations, against 36
// bytes for the same 16 with one column x 8 tokens per thread, which fills the LDS return path.
// The chunks, the unmasked runs and the diagonal's selects are as in k_pf_pv.
template <int HD>
__global__ __launch_bounds__(QMH_WG) void k_pf_pv_rb(const float *__restrict__ att, const float *__restrict__ V,
                                                     float *out, int P, int pos0, int n_heads, int n_kv, int max_seq,
                                                     int8_t *xc, float *xd, int PP, int perm8) {
    constexpr int T = 2048 / HD, VC = QMH_PF_VC;     // tokens per workgroup, positions per chunk
    constexpr int VR = VC * HD / 4 / QMH_WG;          // float4 of V per thread per chunk
    constexpr int PR = T * VC / QMH_WG;               // probabilities per thread per chunk
    __shared__ __align__(16) float ps[VC * T];        // [t][token]
    __shared__ __align__(16) float vs[VC * HD];       // [t][column]
    // token groups by quadrant of blockIdx.y, the odd quadrants reversed: the workgroups that share
    // a CU (y = g, g + ng/4, g + ng/2, g + 3ng/4 when all are resident at once) then carry equal
    // work in sum (late groups see more positions)
    const int ng = gridDim.y, q4 = ng / 4, gy = blockIdx.y;
    const int grp = (ng % 4 == 0 && (gy / q4) % 2 == 1) ? (gy / q4) * q4 + (q4 - 1 - gy % q4) : gy;
    const int h = blockIdx.x, p0 = grp * T, np = min(T, P - p0);
    const int kvh = h / (n_heads / n_kv), kvd = HD * n_kv, tid = threadIdx.x;
    const int tmax = pos0 + p0 + np;  // positions 0 .. tmax-1 are used by some token
    const int tall = pos0 + p0 + 1;   // positions 0 .. tall-1 are used by every token of the group
    const float *vbase = V + (size_t)kvh * HD;
    pf_v4f vr[VR];  // a vector type: float4 copies became memcpys through a stack slot
    float pr[PR];
#define PV_RB_LOAD(C0)                                                                                       \
    _Pragma("unroll") for (int k = 0; k < VR; k++) {                                                         \
        const int e = k * QMH_WG + tid, t = e / (HD / 4), c4 = e % (HD / 4);                                 \
        const int tc = (C0) + t < tmax ? (C0) + t : tmax - 1;                                                \
        vr[k] = *(const pf_v4f *)(vbase + (size_t)tc * kvd + 4 * c4);                                        \
    }                                                                                                        \
    _Pragma("unroll") for (int k = 0; k < PR; k++) {                                                         \
        const int e = k * QMH_WG + tid, kk = e / VC, t = (C0) + e % VC;                                      \
        pr[k] = (kk < np && t <= pos0 + p0 + kk) ? att[((size_t)h * P + p0 + kk) * max_seq + t] : 0.0f;      \
    }
    const int tg = tid / (HD / 2), cg = tid % (HD / 2);  // tokens 4*tg .. +3, columns 2*cg, 2*cg + 1
    float acc[4][2];
#pragma unroll
    for (int a = 0; a < 4; a++) acc[a][0] = acc[a][1] = 0.0f;
    PV_RB_LOAD(0)
    for (int c0 = 0; c0 < tmax; c0 += VC) {
        __syncthreads();
#pragma unroll
        for (int k = 0; k < VR; k++) {
            const int e = k * QMH_WG + tid;
            *(pf_v4f *)(vs + (e / (HD / 4)) * HD + 4 * (e % (HD / 4))) = vr[k];
        }
#pragma unroll
        for (int k = 0; k < PR; k++) {
            const int e = k * QMH_WG + tid;
            ps[(e % VC) * T + e / VC] = pr[k];
        }
        if (c0 + VC < tmax) {
            PV_RB_LOAD(c0 + VC)
        }
        __syncthreads();
        const int nt = min(VC, tmax - c0);
        const int nall = min(nt, max(tall - c0, 0));  // positions of this chunk every token sees
        const float *pp = ps + 4 * tg, *vp = vs + 2 * cg;
        int t = 0;
        for (; t + 4 <= nall; t += 4) {
            float4 pa[4];
            float2 vv[4];
#pragma unroll
            for (int u = 0; u < 4; u++) {
                pa[u] = *(const float4 *)(pp + (t + u) * T);
                vv[u] = *(const float2 *)(vp + (t + u) * HD);
            }
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const float pk[4] = {pa[u].x, pa[u].y, pa[u].z, pa[u].w};
#pragma unroll
                for (int a = 0; a < 4; a++) {
                    acc[a][0] = acc[a][0] + pk[a] * vv[u].x;
                    acc[a][1] = acc[a][1] + pk[a] * vv[u].y;
                }
            }
        }
        for (; t < nt; t++) {
            const float4 p4 = *(const float4 *)(pp + t * T);
            const float2 v2 = *(const float2 *)(vp + t * HD);
            const float pk[4] = {p4.x, p4.y, p4.z, p4.w};
            const int kmin = c0 + t - (pos0 + p0);  // tokens kk >= kmin see position c0 + t
#pragma unroll
            for (int a = 0; a < 4; a++) {
                const bool on = 4 * tg + a >= kmin;
                const float n0 = acc[a][0] + pk[a] * v2.x, n1 = acc[a][1] + pk[a] * v2.y;
                acc[a][0] = on ? n0 : acc[a][0];
                acc[a][1] = on ? n1 : acc[a][1];
            }
        }
    }
#pragma unroll
    for (int a = 0; a < 4; a++) {
        const int kk = 4 * tg + a;
        if (kk < np) {
            float *o = out + (size_t)(p0 + kk) * n_heads * HD + h * HD + 2 * cg;
            o[0] = acc[a][0];
            o[1] = acc[a][1];
        }
    }
    if (xc) {  // uniform
        // Wo's input as its Q8_0 image (the quantizer's steps, src/quant.c:27-52): block b of a token
        // is columns 32*(cg/16) .. +31 of the head, held by the 16 lanes of cg/16 (values 2j, 2j+1 of
        // the block in lane j = cg % 16): amax over those lanes, the fp16 scale, the codes. Q4_0
        // consumers take each 8-group as e0 e2 e4 e6 e1 e3 e5 e7: lane j's two codes are bytes j % 4
        // and 4 + j % 4 of group j / 4.
        const int j = cg & 15, b = h * (HD / 32) + (cg >> 4);
#pragma unroll
        for (int a = 0; a < 4; a++) {
            const int kk = 4 * tg + a;
            float m = 0.0f;
#pragma unroll
            for (int c = 0; c < 2; c++) {
                const float av = fabsf(acc[a][c]);
                m = av > m ? av : m;
            }
#pragma unroll
            for (int o = 1; o < 16; o <<= 1) {
                const float t = __shfl_xor(m, o);
                m = t > m ? t : m;
            }
            const float dd = qmh_h2f(qmh_f2h(qmh_div127(m)));
            const float v4[4] = {acc[a][0], acc[a][1], 0.0f, 0.0f};
            int q[4];
            qmh_q8_codes4(v4, dd, qmh_rcp(dd), q);
            const uint32_t c0 = (uint32_t)q[0] & 0xffu, c1 = (uint32_t)q[1] & 0xffu;
            int8_t *blk = xc + ((size_t)b * PP + p0 + kk) * 32;
            if (perm8) {
                uint32_t w0 = c0 << (8 * (j & 3)), w1 = c1 << (8 * (j & 3));
                w0 |= (uint32_t)__shfl_xor((int)w0, 1);
                w1 |= (uint32_t)__shfl_xor((int)w1, 1);
                w0 |= (uint32_t)__shfl_xor((int)w0, 2);
                w1 |= (uint32_t)__shfl_xor((int)w1, 2);
                if (kk < np && (j & 3) == 0) *(uint2 *)(blk + 8 * (j >> 2)) = make_uint2(w0, w1);
            } else {
                uint32_t w = (c0 | (c1 << 8)) << (16 * (j & 1));
                w |= (uint32_t)__shfl_xor((int)w, 1);
                if (kk < np && (j & 1) == 0) *(uint32_t *)(blk + 2 * j) = w;
            }
            if (kk < np && j == 0) xd[(size_t)b * PP + p0 + kk] = dd;
        }
    }
#undef PV_RB_LOAD
}

extern "C" int qmh_launch_pf_attention(const float *Q, const float *Kt, const float *V, float *att, float *out, int P,
                                       int pos0, int n_heads, int n_kv, int hd, int max_seq, float scale, int8_t *xc,
                                       float *xd, int PP, int perm8, void *stream) {
    if (hd > 128 || hd % 4 || pos0 + P > max_seq || P < 1) return (int)hipErrorInvalidValue;
    // the output's quantized image comes only from the register-blocked P.V (head_dim 128 or 64)
    if (xc && (!xd || (hd != 128 && hd != 64) || P > PP)) return (int)hipErrorInvalidValue;
    hipStream_t s = (hipStream_t)stream;
    const int ng = (P + QMH_PF_TOK - 1) / QMH_PF_TOK, nz = (pos0 + P + QMH_WG - 1) / QMH_WG;
    const dim3 gt(n_heads, (P + 63) / 64, (pos0 + P + 63) / 64);
    if (hd == 128)
        hipLaunchKernelGGL(k_pf_scores_rb<128>, gt, dim3(QMH_WG), 0, s, Q, Kt, att, P, pos0, n_heads, n_kv, max_seq,
                           scale);
    else if (hd == 64)
        hipLaunchKernelGGL(k_pf_scores_rb<64>, gt, dim3(QMH_WG), 0, s, Q, Kt, att, P, pos0, n_heads, n_kv, max_seq,
                           scale);
    else
        hipLaunchKernelGGL(k_pf_scores, dim3(n_heads, ng, nz), dim3(QMH_WG), 0, s, Q, Kt, att, P, pos0, n_heads, n_kv,
                           hd, max_seq, scale);
    const dim3 gs(n_heads, (P + QMH_WG / 64 - 1) / (QMH_WG / 64));
    const int rlen = pos0 + P;  // the longest row
    if (rlen <= 64 * 4) hipLaunchKernelGGL(k_pf_softmax_r<4>, gs, dim3(QMH_WG), 0, s, att, P, pos0, max_seq);
    else if (rlen <= 64 * 8) hipLaunchKernelGGL(k_pf_softmax_r<8>, gs, dim3(QMH_WG), 0, s, att, P, pos0, max_seq);
    else if (rlen <= 64 * 16) hipLaunchKernelGGL(k_pf_softmax_r<16>, gs, dim3(QMH_WG), 0, s, att, P, pos0, max_seq);
    else hipLaunchKernelGGL(k_pf_softmax, gs, dim3(QMH_WG), 0, s, att, P, pos0, max_seq);
    if (hd == 128)
        hipLaunchKernelGGL(k_pf_pv_rb<128>, dim3(n_heads, (P + 15) / 16), dim3(QMH_WG), 0, s, att, V, out, P, pos0,
                           n_heads, n_kv, max_seq, xc, xd, PP, perm8);
    else if (hd == 64)
        hipLaunchKernelGGL(k_pf_pv_rb<64>, dim3(n_heads, (P + 31) / 32), dim3(QMH_WG), 0, s, att, V, out, P, pos0,
                           n_heads, n_kv, max_seq, xc, xd, PP, perm8);
    else
        hipLaunchKernelGGL(k_pf_pv, dim3(n_heads, ng), dim3(QMH_WG), 0, s, att, V, out, P, pos0, n_heads, n_kv, hd,
                           max_seq);
    return (int)hipGetLastError();
}
