// gfx950 attention for batched decode: B independent sequences, one query each, every sequence over
// its own KV cache up to its own position. Per (sequence, head) the arithmetic is that of the single-
// sequence decode (src/model.c:127-156): each score is one lane's serial float chain over head_dim
// times the scale, the softmax is the reference's (src/ops.c:100-112, double sum through the
// certified tree bound or the serial fallback), and each output element is one lane's chain over
// positions 0..pos of p_t * v_t[i] from +0. Kept in its own code object so the decode kernels'
// placement does not move.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "qmh_device.h"
#include "qmh_launch.h"

namespace {

// scores of sequence blockIdx.y, head blockIdx.x, positions blockIdx.z*QMH_WG + threadIdx.x
__global__ __launch_bounds__(QMH_WG) void k_bt_scores(const float *__restrict__ Q, const float *__restrict__ Kt,
                                                      long long kv_stride, const int32_t *__restrict__ pos_arr,
                                                      float *att, int n_heads, int n_kv, int hd, int max_seq,
                                                      float scale) {
    __shared__ float qs[256];
    const int h = blockIdx.x, b = blockIdx.y, t = blockIdx.z * QMH_WG + threadIdx.x;
    const int pos = pos_arr[b];
    if ((int)blockIdx.z * QMH_WG > pos) return;  // past this sequence's positions
    const int kvh = h / (n_heads / n_kv), D = n_heads * hd;
    for (int i = threadIdx.x; i < hd; i += QMH_WG) qs[i] = Q[(size_t)b * D + h * hd + i];
    __syncthreads();
    if (t > pos) return;
    const float *kc = Kt + (size_t)b * kv_stride + (size_t)kvh * hd * max_seq + t;
    float s = 0.0f;
    for (int d0 = 0; d0 < hd; d0 += 64) {  // 64 loads in flight
        float kv[64];
#pragma unroll
        for (int j = 0; j < 64; j++) kv[j] = kc[(size_t)(d0 + j < hd ? d0 + j : hd - 1) * max_seq];
#pragma unroll
        for (int j = 0; j < 64; j++)
            if (d0 + j < hd) s = s + qs[d0 + j] * kv[j];
    }
    att[((size_t)b * n_heads + h) * max_seq + t] = s * scale;
}

// softmax of the row of (sequence blockIdx.y, head blockIdx.x) in place, as the decode kernels
__global__ __launch_bounds__(QMH_WG) void k_bt_softmax(float *att, const int32_t *__restrict__ pos_arr, int n_heads,
                                                       int max_seq) {
    __shared__ double red[16];
    __shared__ float redf[16];
    const int h = blockIdx.x, b = blockIdx.y, n = pos_arr[b] + 1;
    float *x = att + ((size_t)b * n_heads + h) * max_seq;
    const float x0 = x[0];  // read before any thread overwrites it with its exponential
    float m = -__builtin_inff();
    for (int t = threadIdx.x; t < n; t += QMH_WG) m = x[t] > m ? x[t] : m;
    m = qmh_block_max(m, redf);
    if (x0 != x0) m = x0;  // the reference's scan starts from x[0]: a NaN there stays
    double sum = 0.0;
    for (int t = threadIdx.x; t < n; t += QMH_WG) {
        const float e = qmh_expf(x[t] - m);
        x[t] = e;
        sum += (double)e;
    }
    sum = qmh_block_sum_d(sum, red);
    const double d = qmh_sum_slack(sum, n);
    float inv = qmh_recip_of_sum(sum - d);
    if (inv != qmh_recip_of_sum(sum + d)) {  // uniform; serial sum as the reference
        if (threadIdx.x == 0) {
            double ser = 0.0;
            for (int t = 0; t < n; t++) ser += (double)x[t];
            red[8] = ser;
        }
        __syncthreads();
        inv = qmh_recip_of_sum(red[8]);
    }
    for (int t = threadIdx.x; t < n; t += QMH_WG) x[t] = x[t] * inv;
}

// out[b][h*hd + i] = +0 + p_0 v_0[i] + ... + p_pos v_pos[i]: thread i < hd runs column i's chain.
// V passes through LDS 64 positions at a time (cooperative float4 loads; the next chunk is held in
// registers while the current one is used), the probabilities with it.
constexpr int BT_VC = 64;
__global__ __launch_bounds__(QMH_WG) void k_bt_pv(const float *__restrict__ att, const float *__restrict__ V,
                                                  long long kv_stride, const int32_t *__restrict__ pos_arr,
                                                  float *out, int n_heads, int n_kv, int hd, int max_seq) {
    __shared__ __align__(16) float vs[BT_VC * 128];  // [t][column]
    __shared__ float ps[BT_VC];
    const int h = blockIdx.x, b = blockIdx.y, tid = threadIdx.x, n = pos_arr[b] + 1;
    const int kvh = h / (n_heads / n_kv), kvd = hd * n_kv, hd4 = hd >> 2;
    const float *prow = att + ((size_t)b * n_heads + h) * max_seq;
    const float *vbase = V + (size_t)b * kv_stride + (size_t)kvh * hd;
    constexpr int VR = BT_VC * 32 / QMH_WG;  // float4 slots per thread per chunk (32 per row)
    float4 vr[VR];
    float pr = 0.0f;
    auto load = [&](int c0) {
#pragma unroll
        for (int k = 0; k < VR; k++) {
            const int e = k * QMH_WG + tid, t = e >> 5, c4 = e & 31;
            const int tc = c0 + t < n ? c0 + t : n - 1;
            vr[k] = c4 < hd4 ? *(const float4 *)(vbase + (size_t)tc * kvd + 4 * c4) : make_float4(0.f, 0.f, 0.f, 0.f);
        }
        if (tid < BT_VC) pr = c0 + tid < n ? prow[c0 + tid] : 0.0f;
    };
    float acc = 0.0f;
    load(0);
    for (int c0 = 0; c0 < n; c0 += BT_VC) {
        __syncthreads();
#pragma unroll
        for (int k = 0; k < VR; k++) {
            const int e = k * QMH_WG + tid;
            *(float4 *)(vs + (e >> 5) * 128 + 4 * (e & 31)) = vr[k];
        }
        if (tid < BT_VC) ps[tid] = pr;
        if (c0 + BT_VC < n) load(c0 + BT_VC);
        __syncthreads();
        if (tid < hd) {
            const int nt = min(BT_VC, n - c0);
            for (int t = 0; t < nt; t++) acc = acc + ps[t] * vs[t * 128 + tid];
        }
    }
    if (tid < hd) out[(size_t)b * n_heads * hd + h * hd + tid] = acc;
}

// The three steps above in one workgroup per (head blockIdx.x, sequence blockIdx.y), for contexts
// of at most BT_FUSE_MAX positions: the scores and then the probabilities stay in LDS (P), V
// passes through LDS BT_FC positions at a time as the products p_t * v_t (chunk 0 is loaded
// before the scores start, chunk c+1 while chunk c is added). The sums are the same chains in the
// same order.
constexpr int BT_T = 1024;
constexpr int BT_FC = 128;
constexpr int BT_FUSE_MAX = 16384;
constexpr int BT_DECODE_B = 3;
__global__ __launch_bounds__(BT_T, 8) void k_bt_attn(const float *__restrict__ Q, const float *__restrict__ Kt,
                                                  const float *__restrict__ V, long long kv_stride,
                                                  const int32_t *__restrict__ pos_arr, float *out, int n_heads,
                                                  int n_kv, int hd, int max_seq, float scale) {
    extern __shared__ __align__(16) float bt_smem[];
    float *vs = bt_smem;               // [BT_FC][128] staged V rows
    float *P = bt_smem + BT_FC * 128;  // [n] scores, exponentials, probabilities
    __shared__ float qs[128];
    __shared__ float redf[BT_T / 64];
    __shared__ double red[BT_T / 64 + 1];
    const int h = blockIdx.x, b = blockIdx.y, tid = threadIdx.x, n = pos_arr[b] + 1;
    const int kvh = h / (n_heads / n_kv), kvd = hd * n_kv, hd4 = hd >> 2;
    const float *vbase = V + (size_t)b * kv_stride + (size_t)kvh * hd;
    constexpr int VR = BT_FC * 32 / BT_T;  // float4 slots per thread per chunk (32 per row)
    float4 vr[VR];
    auto load = [&](int c0) {
#pragma unroll
        for (int k = 0; k < VR; k++) {
            const int e = k * BT_T + tid, t = e >> 5, c4 = e & 31;
            const int tc = c0 + t < n ? c0 + t : n - 1;
            vr[k] = c4 < hd4 ? *(const float4 *)(vbase + (size_t)tc * kvd + 4 * c4) : make_float4(0.f, 0.f, 0.f, 0.f);
        }
    };
    load(0);
    if (tid < hd) qs[tid] = Q[(size_t)b * n_heads * hd + h * hd + tid];
    __syncthreads();
    // scores: position t is lane t's chain over head_dim (32 K loads in flight: with the V registers
    // the kernel fits 64 VGPRs, so two workgroups share a CU)
    const float *kc = Kt + (size_t)b * kv_stride + (size_t)kvh * hd * max_seq;
    for (int t0 = 0; t0 < n; t0 += BT_T) {
        if (t0 + (tid & ~63) >= n) break;  // whole wave past the context
        const int t = t0 + tid, tc = t < n ? t : n - 1;
        float s = 0.0f;
        for (int d0 = 0; d0 < hd; d0 += 32) {
            float kv[32];
#pragma unroll
            for (int j = 0; j < 32; j++) kv[j] = kc[(size_t)(d0 + j < hd ? d0 + j : hd - 1) * max_seq + tc];
#pragma unroll
            for (int j = 0; j < 32; j++)
                if (d0 + j < hd) s = s + qs[d0 + j] * kv[j];
        }
        if (t < n) P[t] = s * scale;
    }
    __syncthreads();
    // softmax (src/ops.c:100-112) as k_bt_softmax
    const float x0 = P[0];  // read before any thread overwrites it with its exponential
    float m = -__builtin_inff();
    for (int t = tid; t < n; t += BT_T) m = P[t] > m ? P[t] : m;
    m = qmh_block_max(m, redf);
    if (x0 != x0) m = x0;
    double sum = 0.0;
    for (int t = tid; t < n; t += BT_T) {
        const float e = qmh_expf(P[t] - m);
        P[t] = e;
        sum += (double)e;
    }
    sum = qmh_block_sum_d(sum, red);
    const double d = qmh_sum_slack(sum, n);
    float inv = qmh_recip_of_sum(sum - d);
    if (inv != qmh_recip_of_sum(sum + d)) {  // uniform; serial sum as the reference
        if (tid == 0) {
            double ser = 0.0;
            for (int t = 0; t < n; t++) ser += (double)P[t];
            red[BT_T / 64] = ser;
        }
        __syncthreads();
        inv = qmh_recip_of_sum(red[BT_T / 64]);
    }
    for (int t = tid; t < n; t += BT_T) P[t] = P[t] * inv;
    // P·V: every thread stages the products p_t * v_t of its V float4 (the rounded products the
    // chain would form), then lane i < hd runs column i's chain of adds over the chunk
    float acc = 0.0f;
    for (int c0 = 0; c0 < n; c0 += BT_FC) {
        __syncthreads();  // P final (first chunk); the previous chunk's reads done
#pragma unroll
        for (int k = 0; k < VR; k++) {
            const int e = k * BT_T + tid, t = e >> 5;
            const float p = P[c0 + t < n ? c0 + t : n - 1];
            const float4 v = vr[k];
            *(float4 *)(vs + t * 128 + 4 * (e & 31)) = make_float4(p * v.x, p * v.y, p * v.z, p * v.w);
        }
        if (c0 + BT_FC < n) load(c0 + BT_FC);
        __syncthreads();
        if (tid < hd) {
            const int nt = min(BT_FC, n - c0);
            for (int t = 0; t < nt; t++) acc = acc + vs[t * 128 + tid];
        }
    }
    if (tid < hd) out[(size_t)b * n_heads * hd + h * hd + tid] = acc;
}

}  // namespace

extern "C" int qmh_launch_bt_attention(const float *Q, const float *Kt, const float *V, long long kv_stride,
                                       const int32_t *pos, int max_pos, float *att, float *out, int B, int n_heads,
                                       int n_kv, int hd, int max_seq, float scale, int split, void *stream) {
    if (B < 1 || hd < 4 || hd > 128 || hd % 4 || n_kv < 1 || n_heads % n_kv || max_pos < 0 || max_pos >= max_seq)
        return (int)hipErrorInvalidValue;
    hipStream_t s = (hipStream_t)stream;
    // up to BT_DECODE_B sequences: the single-sequence decode kernels with a sequence dimension (MHA
    // shapes), whose workgroups each read a slice of a head's K or V instead of all of it
    if (split == 0 && B <= BT_DECODE_B) {
        const int rc = qmh_launch_attn_batch(Q, Kt, V, kv_stride, pos, att, out, B, n_heads, n_kv, hd, max_seq, scale,
                                             stream);
        if (rc != (int)hipErrorNotSupported) return rc;
    }
    if (split != 1 && max_pos < BT_FUSE_MAX) {
        const size_t lds = (size_t)(BT_FC * 128 + max_pos + 1) * sizeof(float);
        hipLaunchKernelGGL(k_bt_attn, dim3(n_heads, B), dim3(BT_T), lds, s, Q, Kt, V, kv_stride, pos, out, n_heads,
                           n_kv, hd, max_seq, scale);
        return (int)hipGetLastError();
    }
    const int nz = max_pos / QMH_WG + 1;
    hipLaunchKernelGGL(k_bt_scores, dim3(n_heads, B, nz), dim3(QMH_WG), 0, s, Q, Kt, kv_stride, pos, att, n_heads,
                       n_kv, hd, max_seq, scale);
    hipLaunchKernelGGL(k_bt_softmax, dim3(n_heads, B), dim3(QMH_WG), 0, s, att, pos, n_heads, max_seq);
    hipLaunchKernelGGL(k_bt_pv, dim3(n_heads, B), dim3(QMH_WG), 0, s, att, V, kv_stride, pos, out, n_heads, n_kv, hd,
                       max_seq);
    return (int)hipGetLastError();
}

namespace {

// first index of the maximum of row blockIdx.x (src/sampler.c:27-32), then the sequence's next
// token and position for the device greedy loop; record[step*B + b] = idx when record != NULL
template <bool VEC>
__global__ __launch_bounds__(1024) void k_bt_argmax(const float *__restrict__ logits, int V, int32_t *tok,
                                                    int32_t *pos, int32_t *record, int step) {
    __shared__ float bv[16];
    __shared__ int bi[16];
    const int b = blockIdx.x, B = gridDim.x;
    const int idx = qmh_block_argmax<VEC>(logits + (size_t)b * V, V, bv, bi);
    if (threadIdx.x == 0) {
        tok[b] = idx;
        pos[b] += 1;
        if (record) record[(size_t)step * B + b] = idx;
    }
}

}  // namespace

extern "C" int qmh_launch_bt_argmax(const float *logits, int B, int V, int32_t *tok, int32_t *pos, int32_t *record,
                                    int step, void *stream) {
    // 16-byte loads when every row starts 16-byte aligned
    if (((uintptr_t)logits & 15) == 0 && (V % 4 == 0 || B == 1))
        hipLaunchKernelGGL(k_bt_argmax<true>, dim3(B), dim3(1024), 0, (hipStream_t)stream, logits, V, tok, pos, record,
                           step);
    else
        hipLaunchKernelGGL(k_bt_argmax<false>, dim3(B), dim3(1024), 0, (hipStream_t)stream, logits, V, tok, pos,
                           record, step);
    return (int)hipGetLastError();
}
