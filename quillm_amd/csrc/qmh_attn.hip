// gfx950 attention kernels of the quillm token loop (decode: one query position).
//
// Reference src/model.c:127-156, per head h (kv head h/group):
//   att[t] = dot_f32(q_h, K[t]) * scale      serial fp32 dot over head_dim (src/kernels_scalar.c:6-10)
//   softmax(att[0..pos])                     max, expf, double sum, * (float)(1/sum) (src/ops.c:100-112)
//   out[i] = +0; out[i] = out[i] + att[t]*V[t][i] for t = 0..pos in order
// Both float sums keep that order: a score is one lane's chain over head_dim, an output
// element one lane's chain over positions. The caches are laid out for those chains:
//   K: [kvd][max_seq] per layer (transposed): lanes = positions read consecutive floats;
//   V: [max_seq][kvd] per layer: a position's row is contiguous.
// The softmax's double sum is a tree whose float 1/sum is checked against the serial order's
// error bound (qmh_sum_slack) and recomputed serially when the bound cannot decide it.
#include "qmh_device.h"
#include "qmh_launch.h"

// ============================================================================ scores

#define QMH_SC_T 64  // positions per workgroup (one wave, one position per lane)

// HD > 0: head_dim known at compile time -- all HD loads of a lane are issued before its chain
// starts (maximum bytes in flight); HD == 0: any head_dim, loads in groups of 16. The query
// is read with uniform (scalar) loads: every lane of the wave needs the same q values.
// blockIdx.z: the sequence of a batched decode step (its query, caches at Kt + z*kv_stride, score
// rows and position pos_ptr[z]); 0 for the single sequence.
template <int HD>
__global__ __launch_bounds__(QMH_SC_T) void k_attn_scores(const float *__restrict__ q, const float *__restrict__ Kt,
                                                          float *__restrict__ att, const int32_t *pos_ptr,
                                                          int n_heads, int n_kv, int hd_rt, int max_seq, float scale,
                                                          long long kv_stride) {
    const int hd = HD > 0 ? HD : hd_rt;
    const int z = blockIdx.z;
    q += (size_t)z * n_heads * hd;
    Kt += z * kv_stride;
    att += (size_t)z * n_heads * max_seq;
    const int pos = pos_ptr[z];
    const int t0 = blockIdx.y * QMH_SC_T;
    if (pos < 0 || pos >= max_seq || t0 > pos) return;
    const int kvh = blockIdx.x, group = n_heads / n_kv;
    const int t = t0 + (int)threadIdx.x;
    const int tc = t < max_seq ? t : max_seq - 1;  // in-bounds position for the loads
    const float *kcol = Kt + (size_t)kvh * hd * max_seq + tc;
    if (HD > 0) {
        float kv[HD > 0 ? HD : 1];
#pragma unroll
        for (int i = 0; i < HD; i++) kv[i] = kcol[(size_t)i * max_seq];
        for (int hl = 0; hl < group; hl++) {
            const float *qh = q + (size_t)(kvh * group + hl) * HD;
            float s = 0.0f;
#pragma unroll
            for (int i = 0; i < HD; i++) s = s + qh[i] * kv[i];
            if (t <= pos) att[(size_t)(kvh * group + hl) * max_seq + t] = s * scale;
        }
    } else {
        for (int hl = 0; hl < group; hl++) {
            const float *qh = q + (size_t)(kvh * group + hl) * hd;
            float s = 0.0f;
            for (int i0 = 0; i0 < hd; i0 += 16) {
                float kv[16];
#pragma unroll
                for (int k = 0; k < 16; k++) kv[k] = kcol[(size_t)(i0 + k < hd ? i0 + k : hd - 1) * max_seq];
#pragma unroll
                for (int k = 0; k < 16; k++)
                    if (i0 + k < hd) s = s + qh[i0 + k] * kv[k];
            }
            if (t <= pos) att[(size_t)(kvh * group + hl) * max_seq + t] = s * scale;
        }
    }
}

extern "C" int qmh_launch_attn_scores(const float *q, const float *kcache, float *att, const int32_t *pos_ptr,
                                      int n_heads, int n_kv_heads, int head_dim, int max_seq, float scale, void *stream) {
    dim3 grid(n_kv_heads, (max_seq + QMH_SC_T - 1) / QMH_SC_T);
    hipStream_t s = (hipStream_t)stream;
    // a kv head serving several query heads: the K-tile kernel (qmh_ops.hip)
    if (n_heads > n_kv_heads && max_seq % 4 == 0 && max_seq >= 4 &&
        (head_dim == 128 || head_dim == 64 || head_dim == 48))
        return qmh_launch_attn_scores_tile(q, kcache, att, pos_ptr, n_heads, n_kv_heads, head_dim, max_seq, scale,
                                           stream);
#define QMH_SC(HD) \
    hipLaunchKernelGGL(k_attn_scores<HD>, grid, dim3(QMH_SC_T), 0, s, q, kcache, att, pos_ptr, n_heads, n_kv_heads, \
                       head_dim, max_seq, scale, 0LL)
    if (head_dim == 128) QMH_SC(128);
    else if (head_dim == 64) QMH_SC(64);
    else if (head_dim == 48) QMH_SC(48);
    else QMH_SC(0);
#undef QMH_SC
    return (int)hipGetLastError();
}

// ============================================================================ softmax + V sum

#define QMH_PV_CW 16  // output columns per workgroup

// TC: positions per LDS chunk. 640 when the LDS holds it (group <= 8): a context of up to 640
// positions is then one chunk, every V value of the workgroup requested at once.
// MHA (one query head per kv head): the staged values are the products p_t*v_t, each rounded
// as the reference rounds it, so the chain lanes only add.
// A workgroup takes up to 16 query heads of its kv head (16 lanes per head): a group of g heads
// runs as ceil(g/16) sub-groups, blockIdx.x = kv head * ceil(g/16) + sub-group.
template <int TC, bool MHA>
__device__ __forceinline__ void attn_pv_chunks(const float *__restrict__ att, const float *__restrict__ V,
                                               float *__restrict__ out, const int n, int n_heads, int n_kv, int hd,
                                               int max_seq) {
    constexpr int QMH_PV_TC = TC, QMH_PV_VS = TC + 4;  // V chunk row stride == 4 mod 64 floats
    static_assert(TC % 32 == 0 && TC * QMH_PV_CW % QMH_WG == 0, "whole 32-position steps, whole loads");
    constexpr int SVK = 4;  // first head's scores kept in registers: positions < SVK*256
    static_assert(!MHA || TC <= SVK * QMH_WG, "MHA probabilities of the first chunk come from registers");
    extern __shared__ __align__(16) float pv_smem[];
    const int group = n_heads / n_kv, nsub = (group + 15) >> 4, gsm = group < 16 ? group : 16;
    float *P = pv_smem;                              // [gs][TC] probabilities
    float *Vs = pv_smem + gsm * TC;                  // [CW][TC] the chunk (V or, MHA, p*V), transposed
    __shared__ double red[16];
    __shared__ float redf[16];
    __shared__ float mx_s[16], inv_s[16];
    const int kvh = blockIdx.x / nsub, sub = blockIdx.x % nsub, i0 = blockIdx.y * QMH_PV_CW, kvd = hd * n_kv;
    const int hb = kvh * group + 16 * sub, gs = group - 16 * sub < 16 ? group - 16 * sub : 16;  // heads hb .. +gs-1
    const int lane_h = threadIdx.x / QMH_PV_CW, col = threadIdx.x % QMH_PV_CW;
    const bool chain = lane_h < gs;
    const int colc = i0 + (int)(threadIdx.x % QMH_PV_CW) < hd ? i0 + (int)(threadIdx.x % QMH_PV_CW) : hd - 1;
    constexpr int LPT = QMH_PV_TC * QMH_PV_CW / QMH_WG;  // V loads per thread per chunk
    float acc = 0.0f;
    // the first head's scores (positions tid + 256k), issued first: the statistics wait for them only
    float sv[SVK];
    {
        const float *s0 = att + (size_t)hb * max_seq;
#pragma unroll
        for (int k = 0; k < SVK; k++) {
            const int t = (int)threadIdx.x + k * QMH_WG;
            sv[k] = s0[t < n ? t : 0];
        }
    }
    // a chunk's V values: unconditional, clamped loads, all in flight together (the first
    // chunk's under the softmax statistics); the next chunk's are issued before the current
    // chunk's chain runs
    float vv[LPT];
#define QMH_PV_LOAD(T0)                                                 \
    _Pragma("unroll") for (int k = 0; k < LPT; k++) {                   \
        const int e = k * QMH_WG + threadIdx.x, t = e / QMH_PV_CW;      \
        const int tcl = (T0) + t < n ? (T0) + t : n - 1;                \
        vv[k] = V[(size_t)tcl * kvd + kvh * hd + colc];                 \
    }
    QMH_PV_LOAD(0);
    // softmax statistics per head of the sub-group (src/ops.c:100-112)
    for (int hl = 0; hl < gs; hl++) {
        const float *s = att + (size_t)(hb + hl) * max_seq;
        float xv[SVK];
#pragma unroll
        for (int k = 0; k < SVK; k++) {
            const int t = (int)threadIdx.x + k * QMH_WG;
            xv[k] = hl == 0 ? sv[k] : s[t < n ? t : 0];
        }
        float m = -__builtin_inff();
#pragma unroll
        for (int k = 0; k < SVK; k++)
            if ((int)threadIdx.x + k * QMH_WG < n) m = xv[k] > m ? xv[k] : m;
        for (int t = threadIdx.x + SVK * QMH_WG; t < n; t += QMH_WG) m = s[t] > m ? s[t] : m;
        m = qmh_block_max(m, redf);
        if (s[0] != s[0]) m = s[0];  // the reference's scan starts from x[0]: a NaN there stays
        double sum = 0.0;
#pragma unroll
        for (int k = 0; k < SVK; k++)
            if ((int)threadIdx.x + k * QMH_WG < n) sum += (double)qmh_expf(xv[k] - m);
        for (int t = threadIdx.x + SVK * QMH_WG; t < n; t += QMH_WG) sum += (double)qmh_expf(s[t] - m);
        sum = qmh_block_sum_d(sum, red);
        const double d = qmh_sum_slack(sum, n);
        float inv = qmh_recip_of_sum(sum - d);
        if (inv != qmh_recip_of_sum(sum + d)) {  // uniform: the reference's serial order
            double ser = 0.0;                    // (P is free until the chunk loop below)
            for (int t0 = 0; t0 < n; t0 += QMH_PV_TC) {
                const int nt = min(QMH_PV_TC, n - t0);
                for (int t = threadIdx.x; t < nt; t += QMH_WG) P[t] = qmh_expf(s[t0 + t] - m);
                __syncthreads();
                if (threadIdx.x == 0)
                    for (int t = 0; t < nt; t++) ser += (double)P[t];
                __syncthreads();
            }
            inv = qmh_recip_of_sum(ser);  // meaningful in thread 0, the only writer below
        }
        if (threadIdx.x == 0) {
            mx_s[hl] = m;
            inv_s[hl] = inv;
        }
    }
    __syncthreads();
    for (int t0 = 0; t0 < n; t0 += QMH_PV_TC) {
        const int nt = min(QMH_PV_TC, n - t0);
        // probabilities of the chunk, +0 past nt
        if (MHA && t0 == 0) {
            const float m0 = mx_s[0], inv0 = inv_s[0];
#pragma unroll
            for (int k = 0; k < SVK; k++) {
                const int t = (int)threadIdx.x + k * QMH_WG;
                if (t < QMH_PV_TC) P[t] = t < nt ? qmh_expf(sv[k] - m0) * inv0 : 0.0f;
            }
        } else {
            for (int e = threadIdx.x; e < gs * QMH_PV_TC; e += QMH_WG) {
                const int hl = e / QMH_PV_TC, t = e % QMH_PV_TC;
                float p = 0.0f;
                if (t < nt) p = qmh_expf(att[(size_t)(hb + hl) * max_seq + t0 + t] - mx_s[hl]) * inv_s[hl];
                P[hl * QMH_PV_TC + t] = p;
            }
        }
        if (MHA) __syncthreads();  // the products below read P
#pragma unroll
        for (int k = 0; k < LPT; k++) {
            const int e = k * QMH_WG + threadIdx.x, t = e / QMH_PV_CW, cc = e % QMH_PV_CW;
            Vs[cc * QMH_PV_VS + t] = t < nt ? (MHA ? P[t] * vv[k] : vv[k]) : 0.0f;
        }
        if (t0 + QMH_PV_TC < n) QMH_PV_LOAD(t0 + QMH_PV_TC);
        __syncthreads();
        if (chain) {
            // out = out + p_t*v_t in t order; the chunk is zero past nt (p*0 = +0 and the sum,
            // which started at +0, is never -0, so the extra terms change nothing)
            // 32 positions per step, the next step's LDS reads in flight during this step's adds
            // (TC is a multiple of 32 and the chunk is zero up to TC)
            const float4 *p4 = (const float4 *)(P + lane_h * QMH_PV_TC), *v4 = (const float4 *)(Vs + col * QMH_PV_VS);
            const int n32 = (nt + 31) >> 5;
            float4 pc[8], vc[8];
#pragma unroll
            for (int j = 0; j < 8; j++) {
                if (!MHA) pc[j] = p4[j];
                vc[j] = v4[j];
            }
            for (int k = 0; k < n32; k++) {
                float4 pn[8], vn[8];
                const int kn = k + 1 < n32 ? k + 1 : k;  // the last step re-reads itself
#pragma unroll
                for (int j = 0; j < 8; j++) {
                    if (!MHA) pn[j] = p4[8 * kn + j];
                    vn[j] = v4[8 * kn + j];
                }
#pragma unroll
                for (int j = 0; j < 8; j++) {
                    if (MHA) {  // the products were rounded when staged
                        acc = acc + vc[j].x;
                        acc = acc + vc[j].y;
                        acc = acc + vc[j].z;
                        acc = acc + vc[j].w;
                    } else {
                        acc = acc + pc[j].x * vc[j].x;
                        acc = acc + pc[j].y * vc[j].y;
                        acc = acc + pc[j].z * vc[j].z;
                        acc = acc + pc[j].w * vc[j].w;
                    }
                }
#pragma unroll
                for (int j = 0; j < 8; j++) {
                    if (!MHA) pc[j] = pn[j];
                    vc[j] = vn[j];
                }
            }
        }
        __syncthreads();
    }
    if (chain && i0 + col < hd) out[(size_t)(hb + lane_h) * hd + i0 + col] = acc;
#undef QMH_PV_LOAD
}

template <int TC, bool MHA>
__global__ __launch_bounds__(QMH_WG) void k_attn_pv(const float *__restrict__ att, const float *__restrict__ V,
                                                    float *__restrict__ out, const int32_t *pos_ptr, int n_heads,
                                                    int n_kv, int hd, int max_seq) {
    const int n = *pos_ptr + 1;
    if (n < 1 || n > max_seq) return;  // stale position in device memory: touch nothing
    attn_pv_chunks<TC, MHA>(att, V, out, n, n_heads, n_kv, hd, max_seq);
}

// k_attn_pv_mha past TC positions, up to QMH_PV_LONG: the same sums in the same order, streamed.
// The statistics pass keeps every exponential e_t in LDS (P, n floats). V arrives in pieces of 128
// positions, LA pieces ahead, in registers (thread: positions 64*(2j+u) + tid/4, u < 2, columns
// c .. c+3); the products of piece j+1 are staged into one of two LDS buffers while the chain lanes
// add piece j from the other, one barrier per piece.
#define QMH_PV_LONG 8192
template <int LA>
__device__ __forceinline__ void pv_mha_long(const float *__restrict__ s0, const float *__restrict__ V,
                                            float *__restrict__ out, int n, int h, int kvh, int i0, int hd, int kvd,
                                            float *P, float *Vs2) {
    constexpr int PC = 128, VS = PC + 4;  // positions per piece; staged row stride (4 mod 64 floats)
    static_assert(PC * QMH_PV_CW / 4 == 2 * QMH_WG, "a piece is two float4 loads of every thread");
    __shared__ float wmax[QMH_WG / 64];
    __shared__ double wsum[QMH_WG / 64];
    __shared__ double ser_s;
    __shared__ uint64_t etab[32];
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int c = i0 + 4 * (tid & 3), cc = c <= hd - 4 ? c : hd - 4;
    const float *vcol = V + (size_t)kvh * hd + cc;
    const int npc = (n + PC - 1) / PC;
    float4 vr[LA + 1][2];  // ring of V pieces: piece j in vr[j % (LA + 1)]
    auto vload = [&](int j, float4(&d)[2]) {
#pragma unroll
        for (int u = 0; u < 2; u++) {
            const int t = (2 * j + u) * (QMH_WG / 4) + (tid >> 2), tcl = t < n ? t : n - 1;
            d[u] = *(const float4 *)(vcol + (size_t)tcl * kvd);
        }
    };
    // the first pieces' V, issued before the statistics so they arrive under them
#pragma unroll
    for (int k = 0; k < LA; k++) vload(k < npc ? k : npc - 1, vr[k]);
    const uint64_t etv = tid < 32 ? qmh_exp2_tab[tid] : 0;
    // softmax statistics (src/ops.c:100-112) as k_attn_pv_mha: max (NaN never wins; a NaN at x[0]
    // stays), e_t = expf(x_t - max) kept in P, the double sum as a tree checked against the serial order
    float m = -__builtin_inff();
    for (int t = tid; t < n; t += QMH_WG) {
        const float x = s0[t];
        m = x > m ? x : m;
    }
    m = qmh_wave_max(m);
    if (lane == 0) wmax[wv] = m;
    if (tid < 32) etab[tid] = etv;
    __syncthreads();
    m = wmax[0];
#pragma unroll
    for (int w = 1; w < QMH_WG / 64; w++) m = fmaxf(m, wmax[w]);
    if (s0[0] != s0[0]) m = s0[0];
    double sum = 0.0;
    for (int t = tid; t < n; t += QMH_WG) {
        const float e = qmh_expf_t(s0[t] - m, etab);
        P[t] = e;
        sum += (double)e;
    }
    sum = qmh_wave_sum_d(sum);
    if (lane == 0) wsum[wv] = sum;
    __syncthreads();  // also publishes P
    sum = 0.0;
#pragma unroll
    for (int w = 0; w < QMH_WG / 64; w++) sum += wsum[w];
    const double d = qmh_sum_slack(sum, n);
    float inv = qmh_recip_of_sum(sum - d);
    if (inv != qmh_recip_of_sum(sum + d)) {  // uniform: the reference's serial order
        if (tid == 0) {
            double ser = 0.0;
            for (int t = 0; t < n; t++) ser += (double)P[t];
            ser_s = ser;
        }
        __syncthreads();
        inv = qmh_recip_of_sum(ser_s);
    }
    // products of piece j into buffer b: p_t * v_t, +0 past n (the chain's sum started at +0 and
    // is never -0, so the padding changes nothing)
    auto stage = [&](int j, const float4(&v2)[2], int b) {
        float *buf = Vs2 + (size_t)b * QMH_PV_CW * VS;
#pragma unroll
        for (int u = 0; u < 2; u++) {
            const int tl = u * (QMH_WG / 4) + (tid >> 2), t = j * PC + tl;
            const bool on = t < n;
            const float p = on ? P[t] * inv : 0.0f;
            const float4 v = v2[u];
            float *dst = buf + (size_t)(4 * (tid & 3)) * VS + tl;
            dst[0] = on ? p * v.x : 0.0f;
            dst[VS] = on ? p * v.y : 0.0f;
            dst[2 * VS] = on ? p * v.z : 0.0f;
            dst[3 * VS] = on ? p * v.w : 0.0f;
        }
    };
    const bool chain = tid < QMH_PV_CW;
    float acc = 0.0f;
    stage(0, vr[0], 0);
    __syncthreads();
    // piece j: load piece j+LA, stage piece j+1, chain piece j, barrier. Unrolled by LA+1 so the
    // ring indices are constants.
    // Loads and staging are unconditional (a piece past the end stages zeros into the buffer no chain
    // reads next), and the barrier waits only for LDS: the V loads of the next LA pieces stay in flight.
    auto piece = [&](int j, int r) {  // r = j % (LA + 1)
        vload(j + LA < npc ? j + LA : npc - 1, vr[(r + LA) % (LA + 1)]);
        stage(j + 1, vr[(r + 1) % (LA + 1)], (j + 1) & 1);
        if (chain)  // out = out + p_t*v_t in t order (zeros staged past n change nothing)
            acc = qmh_chain_lds(Vs2 + (size_t)(j & 1) * QMH_PV_CW * VS + (size_t)tid * VS, PC, acc);
        __asm__ volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    };
    int j0 = 0;
    for (; j0 + LA + 1 <= npc; j0 += LA + 1) {
#pragma unroll
        for (int r = 0; r <= LA; r++) piece(j0 + r, r);
    }
#pragma unroll
    for (int r = 0; r < LA; r++)
        if (j0 + r < npc) piece(j0 + r, r);  // uniform
    if (chain && i0 + tid < hd) out[(size_t)h * hd + i0 + tid] = acc;
}

// k_attn_pv_mha's path for contexts of up to TC positions, after its loads: the softmax statistics
// over the head's n scores (sv[k] holds position tid + k*QMH_WG) and the V sum of this workgroup's
// 16 columns (vv[k] holds position k*64 + tid/4, columns i0 + 4*(tid%4) .. +3). x0p points to the
// score of position 0 (the reference's max scan starts from it). etv: expf's table entry tid (< 32).
template <int TC>
__device__ __forceinline__ void pv_short(const float (&sv)[(TC + QMH_WG - 1) / QMH_WG],
                                         float4 (&vv)[TC * QMH_PV_CW / 4 / QMH_WG], uint64_t etv, const float *x0p,
                                         int n, int h, int i0, int hd, float *__restrict__ out, float *pv_smem) {
    constexpr int VS = TC + 4;                       // staged row stride == 4 mod 64 floats
    constexpr int L4 = TC * QMH_PV_CW / 4 / QMH_WG;  // float4 V loads per thread
    constexpr int SK = (TC + QMH_WG - 1) / QMH_WG;   // scores per thread
    constexpr int PC = 128;                          // positions per staged piece
    float *P = pv_smem;       // [TC] exponentials e_t
    float *Vs = pv_smem + TC; // [CW][VS] products, transposed
    __shared__ float wmax[QMH_WG / 64];
    __shared__ double wsum[QMH_WG / 64];
    __shared__ double ser_s;
    __shared__ uint64_t etab[32];
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    // softmax statistics (src/ops.c:100-112): max (NaN never wins; a NaN at x[0] stays),
    // e_t = expf(x_t - max) kept in P, the double sum as a tree checked against the serial order
    if (tid < 32) etab[tid] = etv;  // published by the max's barrier
    float m = -__builtin_inff();
#pragma unroll
    for (int k = 0; k < SK; k++)
        if (tid + k * QMH_WG < n) m = sv[k] > m ? sv[k] : m;
    m = qmh_wave_max(m);
    if (lane == 0) wmax[wv] = m;
    __syncthreads();
    m = wmax[0];
#pragma unroll
    for (int w = 1; w < QMH_WG / 64; w++) m = fmaxf(m, wmax[w]);
    const float x0 = *x0p;
    if (x0 != x0) m = x0;
    double sum = 0.0;
#pragma unroll
    for (int k = 0; k < SK; k++) {
        const int t = tid + k * QMH_WG;
        if (t < n) {
            const float e = qmh_expf_t(sv[k] - m, etab);
            P[t] = e;
            sum += (double)e;
        }
    }
    sum = qmh_wave_sum_d(sum);
    if (lane == 0) wsum[wv] = sum;
    __syncthreads();  // also publishes P
    sum = 0.0;
#pragma unroll
    for (int w = 0; w < QMH_WG / 64; w++) sum += wsum[w];
    const double d = qmh_sum_slack(sum, n);
    float inv = qmh_recip_of_sum(sum - d);
    if (inv != qmh_recip_of_sum(sum + d)) {  // uniform: the reference's serial order
        if (tid == 0) {
            double ser = 0.0;
            for (int t = 0; t < n; t++) ser += (double)P[t];
            ser_s = ser;
        }
        __syncthreads();
        inv = qmh_recip_of_sum(ser_s);
    }
    // products of piece j (positions j*PC ..): this thread's float4s 2j and 2j+1, which the loop
    // below keeps in vv[0], vv[1] (the V registers rotate by two per piece, so one copy of the
    // code serves every piece: the kernel's code stays small, and with it the instruction
    // fetches of every launch); +0 past n (the chain's sum started at +0 and is never -0, so the
    // padding changes nothing)
    auto stage = [&](int j) {
#pragma unroll
        for (int u = 0; u < 2; u++) {
            const int t = (2 * j + u) * (QMH_WG / 4) + (tid >> 2);
            const bool on = t < n;
            const float p = on ? P[t] * inv : 0.0f;
            const float4 v = vv[u];
            float *dst = Vs + (size_t)(4 * (tid & 3)) * VS + t;
            dst[0] = on ? p * v.x : 0.0f;
            dst[VS] = on ? p * v.y : 0.0f;
            dst[2 * VS] = on ? p * v.z : 0.0f;
            dst[3 * VS] = on ? p * v.w : 0.0f;
        }
#pragma unroll
        for (int k = 0; k + 2 < L4; k++) vv[k] = vv[k + 2];
    };
    const int npc = (n + PC - 1) / PC;
    const bool chain = tid < QMH_PV_CW;
    const float4 *v4 = (const float4 *)(Vs + (size_t)(chain ? tid : 0) * VS);
    float acc = 0.0f;
    stage(0);
    __syncthreads();
#pragma nounroll
    for (int j = 0; j < npc; j++) {  // uniform trip count
        if (j + 1 < npc) stage(j + 1);
        if (chain) {
            // out = out + p_t*v_t in t order; the piece's terms are read at once, so the LDS
            // latency is paid once per piece
            float4 vc[PC / 4];
#pragma unroll
            for (int q = 0; q < PC / 4; q++) vc[q] = v4[j * (PC / 4) + q];
#pragma unroll
            for (int q = 0; q < PC / 4; q++) {
                acc = acc + vc[q].x;
                acc = acc + vc[q].y;
                acc = acc + vc[q].z;
                acc = acc + vc[q].w;
            }
        }
        __syncthreads();
    }
    if (chain && i0 + tid < hd) out[(size_t)h * hd + i0 + tid] = acc;
}

// One workgroup per (query head, 16 output columns), head_dim a multiple of 4: its V is that of the
// head's kv head h / (n_heads / n_kv) (the query heads of a group read it from L2). Contexts of up
// to TC positions run here; up to QMH_PV_LONG, pv_mha_long; longer ones, only when every kv head
// serves one query head (the launcher keeps grouped heads within QMH_PV_LONG), attn_pv_chunks. Same
// sums in the same order as the reference, laid out for a shorter critical path:
//   * V is read as float4 (4 columns of one position per thread);
//   * the softmax exponentials e_t stay in LDS (P) from the statistics to the products, and the
//     serial fallback of the sum reads them there;
//   * each reduction takes one barrier (its own LDS buffer);
//   * the products p_t*v_t are staged in pieces of 128 positions: while the chain lanes (the
//     first 16 threads, one output column each) add piece j, the other waves stage piece j+1.
template <int TC>
__global__ __launch_bounds__(QMH_WG) void k_attn_pv_mha(const float *__restrict__ att, const float *__restrict__ V,
                                                        float *__restrict__ out, const int32_t *pos_ptr, int n_heads,
                                                        int n_kv, int hd, int max_seq, long long kv_stride) {
    constexpr int L4 = TC * QMH_PV_CW / 4 / QMH_WG;  // float4 V loads per thread
    constexpr int SK = (TC + QMH_WG - 1) / QMH_WG;   // scores per thread
    static_assert(QMH_PV_CW == 16 && TC % 128 == 0 && (TC * QMH_PV_CW / 4) % QMH_WG == 0, "whole pieces, whole loads");
    extern __shared__ __align__(16) float pv_smem[];
    // blockIdx.z: the sequence of a batched decode step (as in k_attn_scores)
    const int z = blockIdx.z;
    att += (size_t)z * n_heads * max_seq;
    V += z * kv_stride;
    out += (size_t)z * n_heads * hd;
    const int n = pos_ptr[z] + 1;
    if (n < 1 || n > max_seq) return;  // stale position in device memory: touch nothing
    if (n > QMH_PV_LONG) {
        if (n_kv != n_heads) return;  // grouped heads never get here (the launcher's bound on max_seq)
        attn_pv_chunks<TC, true>(att, V, out, n, n_heads, n_heads, hd, max_seq);
        return;
    }
    // grouped heads, n_heads % 8 == 0: workgroups x, x + 8, ... (one XCD: x % 8 of the linear id,
    // gridDim.x being n_heads) take consecutive heads, so a group's query heads read their kv head's
    // V through one or two L2s
    const int bx = (int)blockIdx.x;
    const int h = n_kv != n_heads && (n_heads & 7) == 0 ? (bx & 7) * (n_heads >> 3) + (bx >> 3) : bx;
    if (n > TC) {
        pv_mha_long<3>(att + (size_t)h * max_seq, V, out, n, h, h / (n_heads / n_kv), blockIdx.y * QMH_PV_CW, hd,
                       hd * n_kv, pv_smem, pv_smem + QMH_PV_LONG);
        return;
    }
    const int tid = threadIdx.x;
    const int kvh = h / (n_heads / n_kv), i0 = blockIdx.y * QMH_PV_CW, kvd = hd * n_kv;
    const float *s0 = att + (size_t)h * max_seq;
    // loads: expf's table (oldest, so storing it to LDS below waits for nothing else), the head's
    // scores, then the V float4s (position k*64 + tid/4, columns c .. c+3; columns past hd
    // re-read the last whole float4 and are never stored)
    const uint64_t etv = tid < 32 ? qmh_exp2_tab[tid] : 0;
    float sv[SK];
#pragma unroll
    for (int k = 0; k < SK; k++) {
        const int t = tid + k * QMH_WG;
        sv[k] = s0[t < n ? t : 0];
    }
    const int c = i0 + 4 * (tid & 3), cc = c <= hd - 4 ? c : hd - 4;
    float4 vv[L4];
#pragma unroll
    for (int k = 0; k < L4; k++) {
        const int t = k * (QMH_WG / 4) + (tid >> 2), tcl = t < n ? t : n - 1;
        vv[k] = *(const float4 *)(V + (size_t)tcl * kvd + (size_t)kvh * hd + cc);
    }
    pv_short<TC>(sv, vv, etv, s0, n, h, i0, hd, out, pv_smem);
}

// pv_short for the one-launch kernel: the same statistics, products and sums, with the products of
// every position staged at once (Vs holds the whole context; this thread's exponentials read from
// LDS together, then its 4*L4 products stored), one barrier, and the chain lanes (the first CW
// threads) adding the n products of their column in order without further barriers
// (qmh_chain_lds: float4 reads two sets of 32 ahead of the adds). CW output columns (16 or 8): thread
// tid holds V columns 4*(tid % (CW/4)) .. +3 of positions k*PR + tid / (CW/4), PR = 4*256/CW.
template <int TC, int CW>
__device__ __forceinline__ void pv_short_flow(const float (&sv)[(TC + QMH_WG - 1) / QMH_WG],
                                              float4 (&vv)[TC * CW / 4 / QMH_WG], uint64_t etv,
                                              const float *x0p, int n, int h, int i0, int hd,
                                              float *__restrict__ out, float *pv_smem) {
    constexpr int VS = TC + 4;                      // staged row stride == 4 mod 64 floats
    constexpr int L4 = TC * CW / 4 / QMH_WG;        // float4 V loads per thread
    constexpr int SK = (TC + QMH_WG - 1) / QMH_WG;  // scores per thread
    constexpr int NW = QMH_WG / 64;
    constexpr int TPP = CW / 4, PR = QMH_WG / TPP;  // threads per position, positions per round
    static_assert((CW == 16 || CW == 8) && TC % 32 == 0 && L4 * PR == TC,
                  "every position staged, whole 32-position steps");
    float *P = pv_smem;       // [TC] exponentials e_t
    float *Vs = pv_smem + TC; // [CW][VS] products, transposed
    __shared__ float wmax[NW];
    __shared__ double wsum[NW];
    __shared__ double ser_s;
    __shared__ uint64_t etab[32];
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    // softmax statistics (src/ops.c:100-112), as pv_short
    if (tid < 32) etab[tid] = etv;
    float m = -__builtin_inff();
#pragma unroll
    for (int k = 0; k < SK; k++)
        if (tid + k * QMH_WG < n) m = sv[k] > m ? sv[k] : m;
    m = qmh_wave_max(m);
    if (lane == 0) wmax[wv] = m;
    __syncthreads();
    m = wmax[0];
#pragma unroll
    for (int w = 1; w < NW; w++) m = fmaxf(m, wmax[w]);
    const float x0 = *x0p;
    if (x0 != x0) m = x0;
    double sum = 0.0;
#pragma unroll
    for (int k = 0; k < SK; k++) {
        const int t = tid + k * QMH_WG;
        if (t < n) {
            const float e = qmh_expf_t(sv[k] - m, etab);
            P[t] = e;
            sum += (double)e;
        }
    }
    sum = qmh_wave_sum_d(sum);
    if (lane == 0) wsum[wv] = sum;
    __syncthreads();  // also publishes P
    sum = 0.0;
#pragma unroll
    for (int w = 0; w < NW; w++) sum += wsum[w];
    const double d = qmh_sum_slack(sum, n);
    float inv = qmh_recip_of_sum(sum - d);
    if (inv != qmh_recip_of_sum(sum + d)) {  // uniform: the reference's serial order
        if (tid == 0) {
            double ser = 0.0;
            for (int t = 0; t < n; t++) ser += (double)P[t];
            ser_s = ser;
        }
        __syncthreads();
        inv = qmh_recip_of_sum(ser_s);
    }
    // products p_t*v_t of every position, +0 past n
    float pj[L4];
#pragma unroll
    for (int k = 0; k < L4; k++) {
        const int t = k * PR + tid / TPP;
        pj[k] = t < n ? P[t] : 0.0f;
    }
#pragma unroll
    for (int k = 0; k < L4; k++) {
        const int t = k * PR + tid / TPP;
        const bool on = t < n;
        const float p = pj[k] * inv;
        const float4 v = vv[k];
        float *dst = Vs + (size_t)(4 * (tid % TPP)) * VS + t;
        dst[0] = on ? p * v.x : 0.0f;
        dst[VS] = on ? p * v.y : 0.0f;
        dst[2 * VS] = on ? p * v.z : 0.0f;
        dst[3 * VS] = on ? p * v.w : 0.0f;
    }
    __syncthreads();
    if (tid < CW) {  // out = out + p_t*v_t in t order
        const float acc = qmh_chain_lds(Vs + (size_t)tid * VS, n, 0.0f);
        if (i0 + tid < hd) out[(size_t)h * hd + i0 + tid] = acc;
    }
}

// ============================================================================ one launch per step

// The decode step's whole attention in one launch, for contexts of up to TC positions (two
// instances: TC = 640 for head_dim 48, 64 and 128; TC = 1024 for head_dim 64 and 128, and 48 at
// CW = 8, whose slices of at most 256 positions keep one chain lane per position):
// workgroup (cg, h) owns query head h's output columns CW*cg .. +CW-1 (CW = 16 as k_attn_pv_mha,
// or 8 where that grid fits the device) and computes the scores of a slice of the head's
// positions, [cg*sp, cg*sp + sp) with sp = ceil(n / (head_dim/CW)) rounded up to 4. Its K slice arrives as
// float4s of 4 positions of one dimension (all in flight together), is staged in LDS as rows of
// head_dim + 4 floats (one position per row), and one lane per position runs the score's serial
// chain over head_dim. The scores go to attp[h][t] as 64-bit words (score bits | epoch << 32)
// through agent-scope atomic stores; every workgroup of the head then loads the head's n words
// with agent-scope atomic loads until each carries this launch's epoch, and runs k_attn_pv_mha's
// statistics and V sum on them. A word is written and read whole, so a value is taken only with
// the epoch it was stored with: the exchange needs no barrier and no fence.
// The grid is one-dimensional and the dispatcher places workgroup L on XCD L % 8 (round robin
// from XCD 0, measured on MI355X): XCD x takes the hpx = ceil(n_heads/8) consecutive heads
// x*hpx .. x*hpx + hpx - 1 (workgroups L = x + 8*(j*NCG + cg) for its head j), so a head's
// workgroups share one L2, where a poll finds a word another workgroup stored in about 120 ns
// (measured; across XCDs the exchange took microseconds), and the query heads that share a kv head
// read its K and V through one or two L2s instead of eight (32 heads on 4 kv heads, head_dim 64:
// 11.5 -> 10.4 us per launch at position 600). The
// placement is a matter of speed only: the atomics are coherent across the device. The epoch of layer l is
// sync[0]*n_layers + l + 1; sync[0] counts decode steps (k_embed adds one per step), so no two
// launches of a step, nor of two steps, share one, and attp holds only older epochs when a launch
// starts. Every wait is bounded: past `spin` polls the workgroup sets sync[1] (which the host
// reports as an error) and goes on. skew (0 in use) makes the readers wait for an epoch nobody
// writes, so that a test can run the bounded wait to its end from the host. The host launches at
// most as many workgroups as the device holds at once.
#define QMH_AF_TC 640
#define QMH_AF_TC2 1024
#define QMH_AF_SPIN (1u << 16)
// workgroups of k_attn_fused's grid: 8 XCDs x ceil(n_heads / 8) heads x head_dim/cw
__host__ __device__ __forceinline__ int af_grid(int n_heads, int hd, int cw) { return 8 * ((n_heads + 7) / 8) * (hd / cw); }

template <int HD, int TC, int CW>
__global__ __launch_bounds__(QMH_WG) void k_attn_fused(const float *__restrict__ q, const float *__restrict__ Kt,
                                                       const float *__restrict__ V, float *__restrict__ out,
                                                       uint64_t *attp, const int32_t *pos_ptr, uint32_t *sync,
                                                       int n_heads, int n_kv, int max_seq, float scale, int layer,
                                                       int n_layers, uint32_t spin, uint32_t skew) {
    constexpr int NCG = HD / CW, TPP = CW / 4, PR = QMH_WG / TPP;  // column groups; V: threads per position
    constexpr int SPM = ((TC + NCG - 1) / NCG + 3) / 4 * 4;          // most positions of one slice
    constexpr int KS = HD + 4;                                       // LDS row stride of the K slice
    constexpr int KL4 = (SPM / 4 * HD + QMH_WG - 1) / QMH_WG;        // float4 K loads per thread
    constexpr int L4 = TC * CW / 4 / QMH_WG, SK = (TC + QMH_WG - 1) / QMH_WG;
    static_assert(HD % CW == 0 && SPM <= QMH_WG, "whole column groups; one chain lane per position");
    static_assert(CW == 16 || CW == 8, "16 or 8 output columns per workgroup");
    extern __shared__ __align__(16) float af_smem[];
    __shared__ __align__(16) float qs[HD];
    __shared__ float x0s;
    const int n = *pos_ptr + 1;
    if (n < 1 || n > TC || n > max_seq) {  // the host takes longer contexts elsewhere: flag a stray launch
        if (n > TC && n <= max_seq && blockIdx.x == 0 && threadIdx.x == 0)
            __hip_atomic_store(sync + 1, 2u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return;
    }
    const int tid = threadIdx.x;
    const int hpx = (n_heads + 7) >> 3;  // heads per XCD
    const int xj = (int)(blockIdx.x >> 3), h = (int)(blockIdx.x & 7) * hpx + xj / NCG, cg = xj % NCG;
    if (h >= n_heads) return;  // the grid rounds the heads up to a multiple of 8
    const int kvh = h / (n_heads / n_kv), kvd = HD * n_kv, i0 = cg * CW;
    const uint32_t ep = sync[0] * (uint32_t)n_layers + (uint32_t)layer + 1u, want = ep + skew;
    const int sp = ((n + NCG - 1) / NCG + 3) & ~3, p0 = cg * sp;
    const int np = (n - p0 < sp ? n - p0 : sp) > 0 ? (n - p0 < sp ? n - p0 : sp) : 0;  // positions of the slice
    const int np4 = (np + 3) >> 2, np4d = np4 > 0 ? np4 : 1;
    // loads: q, the K slice (element e: dimension e / np4, positions p0 + 4*(e % np4) .. +3, clamped
    // to a whole float4 inside the cache), expf's table, then V as k_attn_pv_mha
    float4 q4 = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    if (tid < HD / 4) q4 = ((const float4 *)(q + (size_t)h * HD))[tid];
    const float *kb = Kt + (size_t)kvh * HD * max_seq;
    float4 kv[KL4];
#pragma unroll
    for (int k = 0; k < KL4; k++) {
        const int e = k * QMH_WG + tid, d = e / np4d < HD ? e / np4d : HD - 1;
        const int t = p0 + 4 * (e % np4d), tc = t <= max_seq - 4 ? t : max_seq - 4;
        kv[k] = qmh_ld_nt4(kb + (size_t)d * max_seq + tc);
    }
    const uint64_t etv = tid < 32 ? qmh_exp2_tab[tid] : 0;
    // V (position k*PR + tid/TPP, columns c .. c+3), loaded non-temporally right behind K: K's
    // arrival waits only for K (the vector-memory counter retires loads in order), and the barrier
    // after the K slice's staging waits for LDS alone, so V streams under the score chains and the
    // poll (measured on MI355X: the poll's results come back behind V either way)
    const int c = i0 + 4 * (tid % TPP), cc = c <= HD - 4 ? c : HD - 4;
    float4 vv[L4];
    auto vload = [&] {
#pragma unroll
        for (int k = 0; k < L4; k++) {
            const int t = k * PR + tid / TPP, tcl = t < n ? t : n - 1;
            vv[k] = qmh_ld_nt4(V + (size_t)tcl * kvd + (size_t)kvh * HD + cc);
        }
    };
    vload();
    // the slice in LDS, row r = position p0 + r
    float *kt = af_smem;
    if (tid < HD / 4) ((float4 *)qs)[tid] = q4;
#pragma unroll
    for (int k = 0; k < KL4; k++) {
        const int e = k * QMH_WG + tid;
        if (e < np4 * HD) {
            const int d = e / np4d, r = 4 * (e % np4d);
            kt[(r + 0) * KS + d] = kv[k].x;
            kt[(r + 1) * KS + d] = kv[k].y;
            kt[(r + 2) * KS + d] = kv[k].z;
            kt[(r + 3) * KS + d] = kv[k].w;
        }
    }
    __asm__ volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");  // the slice and q in LDS
    // scores: s = +0; s = s + q[i]*k[i] in dimension order, times scale (src/model.c:142-146); the
    // row and q are read from LDS eight float4s ahead of their products
    uint64_t *row = attp + (size_t)h * max_seq;
    if (tid < np) {
        const float4 *kr = (const float4 *)(kt + tid * KS), *qr = (const float4 *)qs;
        float sc = 0.0f;
#pragma unroll
        for (int i0 = 0; i0 < HD / 4; i0 += 8) {
            float4 kk[8], qq[8];
#pragma unroll
            for (int i = 0; i < 8; i++)
                if (i0 + i < HD / 4) {
                    kk[i] = kr[i0 + i];
                    qq[i] = qr[i0 + i];
                }
#pragma unroll
            for (int i = 0; i < 8; i++) {
                if (i0 + i >= HD / 4) break;
                sc = sc + qq[i].x * kk[i].x;
                sc = sc + qq[i].y * kk[i].y;
                sc = sc + qq[i].z * kk[i].z;
                sc = sc + qq[i].w * kk[i].w;
            }
        }
        sc = sc * scale;
        __hip_atomic_store(row + p0 + tid, ((uint64_t)ep << 32) | __float_as_uint(sc), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
    }
    // the head's n scores, each once it carries this launch's epoch
    uint64_t w[SK];
#pragma unroll
    for (int k = 0; k < SK; k++) {
        const int t = tid + k * QMH_WG;
        w[k] = t < n ? __hip_atomic_load(row + t, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : (uint64_t)want << 32;
    }
    for (uint32_t it = 0;; it++) {
        bool ok = true;
#pragma unroll
        for (int k = 0; k < SK; k++) ok &= (uint32_t)(w[k] >> 32) == want;
        if (ok) break;
        if (it >= spin) {
            __hip_atomic_store(sync + 1, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            break;
        }
        __builtin_amdgcn_s_sleep(2);
#pragma unroll
        for (int k = 0; k < SK; k++) {
            const int t = tid + k * QMH_WG;
            if ((uint32_t)(w[k] >> 32) != want)
                w[k] = __hip_atomic_load(row + t, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    float sv[SK];
#pragma unroll
    for (int k = 0; k < SK; k++) sv[k] = __uint_as_float((uint32_t)w[k]);
    if (tid == 0) x0s = sv[0];
    __syncthreads();  // the K slice is dead: its LDS is the V sum's from here
    pv_short_flow<TC, CW>(sv, vv, etv, &x0s, n, h, i0, HD, out, af_smem);
}

// dynamic LDS bytes of k_attn_fused<HD, TC, CW>: the larger of the K slice and the V sum's buffers
static size_t af_lds_bytes(int hd, int tc, int cw) {
    const int ncg = hd / cw, spm = ((tc + ncg - 1) / ncg + 3) / 4 * 4;
    const size_t kslice = (size_t)spm * (hd + 4), pv = (size_t)tc + (size_t)cw * (size_t)(tc + 4);
    return sizeof(float) * (kslice > pv ? kslice : pv);
}

extern "C" int qmh_attn_fused_max_n(int instance) { return instance == 0 ? QMH_AF_TC : instance == 1 ? QMH_AF_TC2 : 0; }

// the kernel of an instance for a head size and column width, or NULL. The 1024-position instance
// needs slices of at most 256 positions (one chain lane each): head_dim / cw >= 4
typedef void (*af_fn)(const float *, const float *, const float *, float *, uint64_t *, const int32_t *, uint32_t *,
                      int, int, int, float, int, int, uint32_t, uint32_t);
template <int CW>
static af_fn af_kernel_cw(int head_dim, int instance) {
    if (instance == 0)
        return head_dim == 128 ? k_attn_fused<128, QMH_AF_TC, CW>
               : head_dim == 64 ? k_attn_fused<64, QMH_AF_TC, CW>
               : head_dim == 48 ? k_attn_fused<48, QMH_AF_TC, CW> : NULL;
    if (instance == 1) {
        if (head_dim == 128) return k_attn_fused<128, QMH_AF_TC2, CW>;
        if (head_dim == 64) return k_attn_fused<64, QMH_AF_TC2, CW>;
        if constexpr (CW == 8)
            if (head_dim == 48) return k_attn_fused<48, QMH_AF_TC2, 8>;
    }
    return NULL;
}
static af_fn af_kernel(int head_dim, int instance, int cw) {
    return cw == 16 ? af_kernel_cw<16>(head_dim, instance) : cw == 8 ? af_kernel_cw<8>(head_dim, instance) : NULL;
}

// the output columns per workgroup k_attn_fused runs a shape with: 8 when the grid of 8-column
// workgroups still fits the device one workgroup per CU (twice the workgroups, each loading half
// the K slice and half the V columns: a workgroup's loads are bound by its own CU, not by HBM,
// while half of the CUs would idle), else 16; 0 for a head size it does not take
extern "C" int qmh_attn_fused_cw(int n_heads, int head_dim) {
    if (!af_kernel(head_dim, 0, 16) || n_heads < 1) return 0;
    int dev = 0, ncu = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
        return 0;
    return (long long)af_grid(n_heads, head_dim, 8) <= (long long)ncu ? 8 : 16;
}

// the number of instances k_attn_fused takes the shape with at column width cw (0, 1: contexts up to
// 640, 2: also up to 1024): head_dim 48, 64 or 128 (the second instance: 64 or 128, and 48 at 8
// columns), max_seq a whole number of float4s, and no more workgroups than the device holds at once
// (every head's workgroups run together)
extern "C" int qmh_attn_fused_supported(int n_heads, int n_kv_heads, int head_dim, int max_seq, int cw) {
    if (max_seq % 4 || max_seq < 4 || n_kv_heads < 1 || n_heads % n_kv_heads || !af_kernel(head_dim, 0, cw)) return 0;
    int dev = 0, ncu = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
        return 0;
    int count = 0;
    for (int i = 0; i < 2; i++) {
        int per = 0;
        const af_fn k = af_kernel(head_dim, i, cw);
        if (!k ||
            hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, (const void *)k, QMH_WG,
                                                         af_lds_bytes(head_dim, qmh_attn_fused_max_n(i), cw)) != hipSuccess ||
            (long long)af_grid(n_heads, head_dim, cw) > (long long)per * ncu)
            break;
        count = i + 1;
    }
    return count;
}

// the caller has checked qmh_attn_fused_supported for the shape, column width and instance; stall !=
// 0 (tests only): the readers wait for an epoch nobody writes, for 64 polls
extern "C" int qmh_launch_attn_fused(const float *q, const float *kcache, const float *vcache, float *out,
                                     uint64_t *attp, const int32_t *pos_ptr, uint32_t *sync, int n_heads,
                                     int n_kv_heads, int head_dim, int max_seq, float scale, int layer, int n_layers,
                                     int instance, int cw, int stall, void *stream) {
    const af_fn k = af_kernel(head_dim, instance, cw);
    if (!k || max_seq % 4 || max_seq < 4 || n_kv_heads < 1 || n_heads % n_kv_heads) return (int)hipErrorNotSupported;
    const dim3 grid(af_grid(n_heads, head_dim, cw));
    const size_t lds = af_lds_bytes(head_dim, qmh_attn_fused_max_n(instance), cw);
    hipStream_t s = (hipStream_t)stream;
    const uint32_t spin = stall ? 64u : QMH_AF_SPIN, skew = stall ? 1u : 0u;
    hipLaunchKernelGGL(k, grid, dim3(QMH_WG), lds, s, q, kcache, vcache, out, attp, pos_ptr, sync, n_heads, n_kv_heads,
                       max_seq, scale, layer, n_layers, spin, skew);
    return (int)hipGetLastError();
}

extern "C" int qmh_launch_attn_pv(const float *att, const float *vcache, float *out, const int32_t *pos_ptr,
                                  int n_heads, int n_kv_heads, int head_dim, int max_seq, void *stream) {
    if (n_kv_heads < 1 || n_heads % n_kv_heads) return (int)hipErrorInvalidValue;
    // k_attn_pv: sub-groups of up to 16 query heads per workgroup (16 lanes each)
    const int group = n_heads / n_kv_heads, nsub = (group + 15) / 16, gsm = group < 16 ? group : 16;
    dim3 grid(n_kv_heads * nsub, (head_dim + QMH_PV_CW - 1) / QMH_PV_CW);
    hipStream_t s = (hipStream_t)stream;
#define QMH_PV_GO(TC, MHA)                                                                                \
    hipLaunchKernelGGL((k_attn_pv<TC, MHA>), grid, dim3(QMH_WG), sizeof(float) * ((size_t)gsm * TC + QMH_PV_CW * (TC + 4)), \
                       s, att, vcache, out, pos_ptr, n_heads, n_kv_heads, head_dim, max_seq)
    if (head_dim % 4 == 0 && (group == 1 || max_seq <= QMH_PV_LONG)) {
        // one workgroup per query head; the larger of the two paths' LDS: the whole-context one
        // (<= 640 positions) and the streamed one (exponentials of up to QMH_PV_LONG positions, two
        // staged pieces of 128)
        const size_t lds_a = (size_t)640 + QMH_PV_CW * (640 + 4), lds_b = (size_t)QMH_PV_LONG + 2 * QMH_PV_CW * (128 + 4);
        hipLaunchKernelGGL(k_attn_pv_mha<640>, dim3(n_heads, grid.y), dim3(QMH_WG),
                           sizeof(float) * (lds_a > lds_b ? lds_a : lds_b), s, att, vcache, out, pos_ptr, n_heads,
                           n_kv_heads, head_dim, max_seq, 0LL);
    }
    else if (group == 1) QMH_PV_GO(640, true);
    else if (group <= 8) QMH_PV_GO(640, false);
    else QMH_PV_GO(256, false);
#undef QMH_PV_GO
    return (int)hipGetLastError();
}

// The decode kernels over B sequences of a batched step (blockIdx.z = sequence): one query head per
// kv head and head_dim 128, 64 or 48. Scores spread over (head, 64 positions) workgroups and P.V
// over (head, 16 columns) ones, where the fused batched kernel reads a head's whole K and V in one
// workgroup. Returns hipErrorNotSupported for other shapes.
extern "C" int qmh_launch_attn_batch(const float *Q, const float *Kt, const float *V, long long kv_stride,
                                     const int32_t *pos, float *att, float *out, int B, int n_heads, int n_kv,
                                     int hd, int max_seq, float scale, void *stream) {
    if (n_heads != n_kv || (hd != 128 && hd != 64 && hd != 48) || B < 1) return (int)hipErrorNotSupported;
    hipStream_t s = (hipStream_t)stream;
    const dim3 gs(n_kv, (max_seq + QMH_SC_T - 1) / QMH_SC_T, B);
    if (hd == 128)
        hipLaunchKernelGGL(k_attn_scores<128>, gs, dim3(QMH_SC_T), 0, s, Q, Kt, att, pos, n_heads, n_kv, hd, max_seq,
                           scale, kv_stride);
    else if (hd == 64)
        hipLaunchKernelGGL(k_attn_scores<64>, gs, dim3(QMH_SC_T), 0, s, Q, Kt, att, pos, n_heads, n_kv, hd, max_seq,
                           scale, kv_stride);
    else
        hipLaunchKernelGGL(k_attn_scores<48>, gs, dim3(QMH_SC_T), 0, s, Q, Kt, att, pos, n_heads, n_kv, hd, max_seq,
                           scale, kv_stride);
    const size_t lds_a = (size_t)640 + QMH_PV_CW * (640 + 4), lds_b = (size_t)QMH_PV_LONG + 2 * QMH_PV_CW * (128 + 4);
    hipLaunchKernelGGL(k_attn_pv_mha<640>, dim3(n_heads, (hd + QMH_PV_CW - 1) / QMH_PV_CW, B), dim3(QMH_WG),
                       sizeof(float) * (lds_a > lds_b ? lds_a : lds_b), s, att, V, out, pos, n_heads, n_kv, hd,
                       max_seq, kv_stride);
    return (int)hipGetLastError();
}
