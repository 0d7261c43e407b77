/* HIP host runtime for the quillm token loop: C11 on the HIP runtime C API.
 *
 * Owns the device, the library stream, device weights (repacked from the reference's row
 * layout), and the device model: one hipGraph per decode step, replayed with the token and
 * position read from device memory, so forward(token, pos) costs one small copy in, one graph
 * launch and one logits copy out, and the greedy loop never returns to the host. */
#define _DEFAULT_SOURCE
#ifndef __HIP_PLATFORM_AMD__
#define __HIP_PLATFORM_AMD__ 1
#endif
#include <hip/hip_runtime_api.h>
#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

#include "../../include/qmhip.h"
#include "../csrc/qmh_launch.h"
#include "qlm_io.h"

int qmh_gen_qlm_impl(const char *path, const qmh_config *cfg, int wtype, uint64_t seed, int n_threads, char *err,
                     size_t errlen);

/* ------------------------------------------------------------------ errors */

static _Thread_local char g_err[512];

static int fail(const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
    return -1;
}

const char *qmh_last_error(void) { return g_err; }

#define HIPCHK(call)                                                                                                  \
    do {                                                                                                              \
        hipError_t e_ = (call);                                                                                       \
        if (e_ != hipSuccess) return fail("%s failed: %s", #call, hipGetErrorString(e_));                            \
    } while (0)
#define LCHK(call)                                                                                                    \
    do {                                                                                                              \
        int e_ = (call);                                                                                              \
        if (e_ != 0) return fail("%s failed: %s", #call, hipGetErrorString((hipError_t)e_));                         \
    } while (0)

/* ------------------------------------------------------------------ runtime */

static int g_ready, g_dev = -1, g_cus = 256;
static hipStream_t g_stream;
static float *g_rope_scratch; /* op-level rope: one position's (cos, sin) pairs */
#define ROPE_SCRATCH_PAIRS 4096

int qmh_available(void) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) return 0;
    for (int i = 0; i < n; i++) {
        hipDeviceProp_t p;
        if (hipGetDeviceProperties(&p, i) == hipSuccess && strncmp(p.gcnArchName, "gfx950", 6) == 0) return 1;
    }
    return 0;
}

int qmh_init(int device) {
    if (g_ready && device == g_dev) return 0;
    if (g_ready) return fail("qmh_init: already initialised on device %d", g_dev);
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= device || device < 0) return fail("no HIP device %d", device);
    hipDeviceProp_t p;
    HIPCHK(hipGetDeviceProperties(&p, device));
    if (strncmp(p.gcnArchName, "gfx950", 6) != 0)
        return fail("device %d is %s; this library is built for gfx950 only", device, p.gcnArchName);
    HIPCHK(hipSetDevice(device));
    HIPCHK(hipStreamCreateWithFlags(&g_stream, hipStreamNonBlocking));
    HIPCHK(hipMalloc((void **)&g_rope_scratch, sizeof(float) * 2 * ROPE_SCRATCH_PAIRS));
    g_cus = p.multiProcessorCount > 0 ? p.multiProcessorCount : 256;
    void *scr = NULL; /* the sampler's static scratch: its address on this device, looked up now */
    LCHK(qmh_sample_scratch(&scr));
    g_dev = device;
    g_ready = 1;
    return 0;
}

static int ensure(void) { return g_ready ? 0 : qmh_init(0); }
static hipStream_t S(void *stream) { return stream ? (hipStream_t)stream : g_stream; }

void *qmh_stream(void) { return ensure() ? NULL : (void *)g_stream; }

void *qmh_dev_alloc(size_t bytes) {
    void *p = NULL;
    if (ensure()) return NULL;
    hipError_t e = hipMalloc(&p, bytes ? bytes : 1);
    if (e != hipSuccess) {
        fail("hipMalloc(%zu): %s", bytes, hipGetErrorString(e));
        return NULL;
    }
    return p;
}
int qmh_dev_free(void *p) {
    if (p) HIPCHK(hipFree(p));
    return 0;
}
int qmh_memcpy_h2d(void *dst, const void *src, size_t bytes) {
    if (ensure()) return -1;
    HIPCHK(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, g_stream));
    HIPCHK(hipStreamSynchronize(g_stream));
    return 0;
}
int qmh_memcpy_d2h(void *dst, const void *src, size_t bytes) {
    if (ensure()) return -1;
    HIPCHK(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, g_stream));
    HIPCHK(hipStreamSynchronize(g_stream));
    return 0;
}
int qmh_memset(void *dst, int value, size_t bytes) {
    if (ensure()) return -1;
    HIPCHK(hipMemsetAsync(dst, value, bytes, g_stream));
    return 0;
}
int qmh_sync(void) {
    if (ensure()) return -1;
    HIPCHK(hipStreamSynchronize(g_stream));
    return 0;
}

/* ------------------------------------------------------------------ op level */

int qmh_fp16_to_fp32(const uint16_t *h, float *f, int64_t n, void *stream) {
    if (ensure()) return -1;
    LCHK(qmh_launch_h2f(h, f, n, S(stream)));
    return 0;
}
int qmh_fp32_to_fp16(const float *f, uint16_t *h, int64_t n, void *stream) {
    if (ensure()) return -1;
    LCHK(qmh_launch_f2h(f, h, n, S(stream)));
    return 0;
}
int qmh_quantize_rows_q8(const float *x, void *y, int64_t rows, int64_t n, void *stream) {
    if (ensure()) return -1;
    LCHK(qmh_launch_quantize_rows(x, y, rows, n, QMH_Q8_0, S(stream)));
    return 0;
}
int qmh_quantize_rows_q4(const float *x, void *y, int64_t rows, int64_t n, void *stream) {
    if (ensure()) return -1;
    LCHK(qmh_launch_quantize_rows(x, y, rows, n, QMH_Q4_0, S(stream)));
    return 0;
}
int qmh_row_to_f32(int dtype, const void *row, float *y, int64_t n, void *stream) {
    if (ensure()) return -1;
    if (!(dtype == QMH_F32 || dtype == QMH_Q8_0 || dtype == QMH_Q4_0)) return fail("bad dtype %d", dtype);
    LCHK(qmh_launch_row_to_f32(row, dtype, y, n, S(stream)));
    return 0;
}
int qmh_rmsnorm(float *out, const float *x, const float *w, int64_t n, float eps, void *stream) {
    if (ensure()) return -1;
    LCHK(qmh_launch_rmsnorm(out, x, w, n, eps, S(stream)));
    return 0;
}
int qmh_softmax(float *x, int64_t n, void *stream) {
    if (ensure()) return -1;
    LCHK(qmh_launch_softmax(x, n, S(stream)));
    return 0;
}
int qmh_swiglu(float *gate, const float *up, int64_t n, void *stream) {
    if (ensure()) return -1;
    LCHK(qmh_launch_swiglu(gate, up, n, S(stream)));
    return 0;
}
int qmh_argmax(const float *x, int32_t n, int32_t *out, void *stream) {
    if (ensure()) return -1;
    if (n < 1) return fail("argmax of an empty vector");
    LCHK(qmh_launch_argmax(x, n, out, NULL, NULL, 0, S(stream)));
    return 0;
}

/* (cos, sin) of position pos for pair i, in the reference's double formula (src/ops.c:116-118),
 * rounded to fp32 on the host so the device rotates with bit-identical factors */
static void rope_pairs(float *out, int64_t head_dim, int64_t pos, float theta) {
    for (int64_t i = 0; i < head_dim / 2; i++) {
        double freq = pow((double)theta, -2.0 * (double)i / (double)head_dim);
        double ang = (double)pos * freq;
        out[2 * i] = (float)cos(ang);
        out[2 * i + 1] = (float)sin(ang);
    }
}

int qmh_rope(float *v, int64_t n_heads, int64_t head_dim, int64_t pos, float theta, void *stream) {
    if (ensure()) return -1;
    if (head_dim / 2 > ROPE_SCRATCH_PAIRS || head_dim < 0 || n_heads < 0) return fail("rope: head_dim too large");
    float cs[2 * ROPE_SCRATCH_PAIRS];
    rope_pairs(cs, head_dim, pos, theta);
    HIPCHK(hipStreamSynchronize(S(stream))); /* scratch is shared by every call */
    HIPCHK(hipMemcpy(g_rope_scratch, cs, sizeof(float) * (size_t)head_dim, hipMemcpyHostToDevice));
    LCHK(qmh_launch_rope(v, n_heads, head_dim, g_rope_scratch, 0, S(stream)));
    HIPCHK(hipStreamSynchronize(S(stream)));
    return 0;
}

int qmh_matmul_nt(const float *A, const float *B, float *C, int64_t M, int64_t N, int64_t K, void *stream) {
    if (ensure()) return -1;
    if (M < 0 || N < 0 || K < 0) return fail("matmul_nt: negative size");
    LCHK(qmh_launch_gemm_nt(A, B, C, M, N, K, S(stream)));
    return 0;
}

/* ------------------------------------------------------------------ device weights */

struct qmh_weight {
    int dtype, tile_r, nb, ntiles;
    int64_t rows, cols; /* rows: output rows (per half for an interleaved pair) */
    void *codes;        /* tiled codes, or row-major f32 */
    uint16_t *scales;
};

static void weight_release(struct qmh_weight *w) {
    if (w->codes) hipFree(w->codes);
    if (w->scales) hipFree(w->scales);
    memset(w, 0, sizeof *w);
}

/* Build a device weight from nsrc host matrices with the same dtype and cols:
 * interleave = 0: rows appended in order (e.g. [wq; wk; wv]), tiles of tile_r (8 or 16) rows;
 * interleave = 1: two matrices of equal rows, tile t holding tile_r/2 rows of each (w1 | w3;
 * tile_r 32 or 64). Small matrices get 8-row tiles: twice the workgroups, so more of the GPU
 * streams them. */
static int weight_build(struct qmh_weight *w, int dtype, int nsrc, const void *const *src, const int64_t *src_rows,
                        int64_t cols, int interleave, int tile_r) {
    memset(w, 0, sizeof *w);
    w->dtype = dtype;
    w->cols = cols;
    w->nb = (int)((cols + 31) / 32);
    int64_t total = 0;
    for (int i = 0; i < nsrc; i++) total += src_rows[i];
    if (dtype == QMH_F32) {
        w->rows = total;
        size_t rb = (size_t)cols * 4;
        HIPCHK(hipMalloc(&w->codes, rb * (size_t)total));
        size_t off = 0;
        for (int i = 0; i < nsrc; i++) {
            HIPCHK(hipMemcpy((uint8_t *)w->codes + off, src[i], rb * (size_t)src_rows[i], hipMemcpyHostToDevice));
            off += rb * (size_t)src_rows[i];
        }
        return 0;
    }
    if (dtype != QMH_Q8_0 && dtype != QMH_Q4_0) return fail("unsupported dtype %d", dtype);
    const int cb = dtype == QMH_Q4_0 ? 16 : 32;
    const size_t rb = qlm_row_bytes(dtype, cols);
    if (interleave) {
        if (nsrc != 2 || src_rows[0] != src_rows[1]) return fail("interleaved weight needs two equal matrices");
        if (tile_r != 32 && tile_r != 64) return fail("unsupported interleaved tile height %d", tile_r);
        w->tile_r = tile_r;
        w->rows = src_rows[0];
        w->ntiles = (int)((src_rows[0] + tile_r / 2 - 1) / (tile_r / 2));
    } else {
        if (tile_r != 8 && tile_r != QMH_TILE_R) return fail("unsupported tile height %d", tile_r);
        w->tile_r = tile_r;
        w->rows = total;
        w->ntiles = (int)((total + tile_r - 1) / tile_r);
    }
    /* + QMH_WEIGHT_PAD_SLOTS: the matvec loads whole chunks unconditionally, so the last chunk
     * of the last tile may read up to one chunk past the tiles (zeros, never used) */
    const size_t slots = (size_t)w->ntiles * (size_t)w->nb * (size_t)w->tile_r + QMH_WEIGHT_PAD_SLOTS;
    HIPCHK(hipMalloc(&w->codes, slots * (size_t)cb));
    HIPCHK(hipMalloc((void **)&w->scales, slots * 2));
    HIPCHK(hipMemsetAsync(w->codes, 0, slots * (size_t)cb, g_stream));
    HIPCHK(hipMemsetAsync(w->scales, 0, slots * 2, g_stream));
    size_t maxb = 0;
    for (int i = 0; i < nsrc; i++) maxb = rb * (size_t)src_rows[i] > maxb ? rb * (size_t)src_rows[i] : maxb;
    void *stage = NULL;
    HIPCHK(hipMalloc(&stage, maxb ? maxb : 1));
    int64_t row_off = 0;
    int rc = 0;
    for (int i = 0; i < nsrc && rc == 0; i++) {
        hipError_t e = hipMemcpyAsync(stage, src[i], rb * (size_t)src_rows[i], hipMemcpyHostToDevice, g_stream);
        if (e == hipSuccess)
            e = (hipError_t)qmh_launch_repack(stage, src_rows[i], w->nb, dtype, w->codes, w->scales, w->tile_r,
                                              row_off, interleave ? i : -1, (int64_t)slots, g_stream);
        if (e == hipSuccess) e = hipStreamSynchronize(g_stream);
        if (e != hipSuccess) rc = fail("weight upload: %s", hipGetErrorString(e));
        row_off += src_rows[i];
    }
    hipFree(stage);
    return rc;
}

qmh_weight *qmh_weight_upload(int dtype, int64_t rows, int64_t cols, const void *host_rows) {
    if (ensure()) return NULL;
    if (rows <= 0 || cols <= 0 || !host_rows) {
        fail("weight_upload: empty matrix");
        return NULL;
    }
    qmh_weight *w = calloc(1, sizeof *w);
    if (!w) return NULL;
    const void *src[1] = {host_rows};
    int64_t r[1] = {rows};
    if (weight_build(w, dtype, 1, src, r, cols, 0, QMH_TILE_R)) {
        weight_release(w);
        free(w);
        return NULL;
    }
    return w;
}

void qmh_weight_free(qmh_weight *w) {
    if (!w) return;
    weight_release(w);
    free(w);
}

/* QMH_EXACT_NORM (tests), read when a model loads: the matvecs' RMSNorms always take the serial
 * sum of squares, the path a failed certificate takes */
static int g_exact_norm;

static void mv_args_for(const struct qmh_weight *w, qmh_mv_args *a) {
    memset(a, 0, sizeof *a);
    a->exact_norm = g_exact_norm;
    a->dtype = w->dtype;
    a->codes = w->codes;
    a->scales = w->scales;
    a->nb = w->nb;
    a->cols = (int)w->cols;
    a->tile_r = w->tile_r;
    a->ntiles = w->ntiles;
    a->rows = (int)w->rows;
}

/* one workgroup per CU; two per CU for matrices of many tiles (the output matrix), whose
 * workgroups would otherwise each stream a long range behind a short prologue */
static int mv_launch(const qmh_mv_args *a, hipStream_t s) {
    if (a->dtype == QMH_F32) return qmh_launch_matvec_f32(a, s);
    const int want = g_cus * (a->ntiles >= 6 * g_cus ? 2 : 1);
    const int grid = qmh_matvec_grid(a->ntiles, a->nb, a->tile_r, a->dtype, want);
    return grid < 1 ? (int)hipErrorInvalidValue : qmh_launch_matvec(a, grid, s);
}

int qmh_matvec(const qmh_weight *W, const float *x, float *y, void *xq, void *stream) {
    if (ensure()) return -1;
    if (!W) return fail("matvec: NULL weight");
    qmh_mv_args a;
    mv_args_for(W, &a);
    a.x = x;
    a.epi = QMH_EPI_STORE;
    a.out0 = y;
    a.xq_out = W->dtype == QMH_F32 ? NULL : (uint8_t *)xq;
    LCHK(mv_launch(&a, S(stream)));
    return 0;
}

int qmh_rmsnorm_matvec(const qmh_weight *W, const float *x, const float *norm_w, float eps, float *y, void *xq,
                       void *stream) {
    if (ensure()) return -1;
    if (!W || !norm_w) return fail("rmsnorm_matvec: NULL weight or gain");
    qmh_mv_args a;
    mv_args_for(W, &a);
    a.x = x;
    a.norm_w = norm_w;
    a.eps = eps;
    a.epi = QMH_EPI_STORE;
    a.out0 = y;
    a.xq_out = W->dtype == QMH_F32 ? NULL : (uint8_t *)xq;
    LCHK(mv_launch(&a, S(stream)));
    return 0;
}

/* ------------------------------------------------------------------ model */

typedef struct {
    struct qmh_weight qkv, wo, w13, w2;
    int w2_image; /* W1|W3 and W2 quantized: W13 writes W2's input as a quantized image (d_hq) */
} dev_layer;

struct qmh_model {
    qmh_config cfg;
    int hd, kvd, group;
    int emb_dtype;
    void *d_embd;
    float *d_norms; /* [2L+1][D]: attn_norm l, ffn_norm l, ..., final norm */
    dev_layer *layers;
    struct qmh_weight output;
    float *d_rope;  /* [max_seq][hd/2][2] */
    float *d_x, *d_xb, *d_q, *d_hb, *d_att, *d_logits, *d_kt, *d_v;
    void *d_hq; /* W2's input quantized (QMH_XQ_IMAGE_BYTES(nb of hidden_dim)) */
    int32_t *d_tokpos; /* token, pos, step, - */
    int32_t *d_record; /* greedy ids [max_seq] */
    int32_t *h_tokpos; /* pinned [max_seq][4] */
    float *h_logits;   /* pinned [vocab] */
    hipGraph_t graph_fwd, graph_greedy;
    hipGraphExec_t exec_fwd, exec_greedy;
    /* the same steps with the attention in one launch (k_attn_fused), instance i for positions
     * below qmh_attn_fused_max_n(i), i < af_n */
    hipGraph_t graph_fwd_af[2], graph_greedy_af[2];
    hipGraphExec_t exec_fwd_af[2], exec_greedy_af[2];
    int af_n;          /* k_attn_fused's instances that take the model's shape (0: none) */
    int af_inst;       /* the instance ST_ATTN launches */
    int af_cw;         /* its output columns per workgroup (16 or 8) */
    int af_stall;      /* QMH_AF_FORCE_STALL (tests): the one-launch attention's waits run out */
    uint64_t *d_attp;  /* [n_heads][max_seq] epoch-tagged scores of k_attn_fused */
    uint32_t *d_sync;  /* [0] decode steps (k_embed), [1] k_attn_fused's wait status */
    uint32_t *h_sync;  /* pinned copy of d_sync[1] */
    int use_graph; /* 0 when QMH_NO_GRAPH is set: the same kernels, enqueued one by one (profiling) */
    /* batched prefill (every matrix quantized): up to pf_cap tokens per pass, padded to pf_pp */
    int pf_ok, pf_cap, pf_pp;
    int32_t *d_pf_tok, *h_pf_tok;
    float *d_pf_x, *d_pf_xb, *d_pf_q, *d_pf_hb, *d_pf_att, *d_pf_logits, *d_pf_xd;
    int8_t *d_pf_xc2; /* W2's input image, written by W1|W3's epilogue past QMH_PF_SKINNY_P tokens */
    float *d_pf_xd2;
    int8_t *d_pf_xc;
};

/* the kernels of one decode step, by stage (which) and layer */
enum { ST_QKV = 0, ST_WO = 1, ST_W13 = 2, ST_W2 = 3, ST_OUT = 4, ST_SCORES = 5, ST_PV = 6, ST_ATTN = 7, ST_COUNT };

static int enqueue_stage(qmh_model *m, int which, int l, hipStream_t s) {
    const qmh_config *c = &m->cfg;
    const int D = c->dim, H = c->hidden_dim, S_ = c->max_seq;
    const int32_t *pos_ptr = m->d_tokpos + 1;
    dev_layer *L = &m->layers[l];
    float *kl = m->d_kt + (size_t)l * S_ * m->kvd, *vl = m->d_v + (size_t)l * S_ * m->kvd;
    qmh_mv_args a;
    switch (which) {
    case ST_QKV: /* xb = rmsnorm(x); q,k,v = W xb; rope(q,k); k,v -> cache (src/model.c:166-173) */
        mv_args_for(&L->qkv, &a);
        a.x = m->d_x;
        a.norm_w = m->d_norms + (size_t)(2 * l) * D;
        a.eps = c->norm_eps;
        a.epi = QMH_EPI_QKV;
        a.out0 = m->d_q;
        a.out1 = kl;
        a.out2 = vl;
        a.seg1 = D;
        a.seg2 = D + m->kvd;
        a.rope = m->d_rope;
        a.pos_ptr = pos_ptr;
        a.head_dim = m->hd;
        a.max_seq = S_;
        a.kvd = m->kvd;
        return mv_launch(&a, s);
    case ST_SCORES: /* src/model.c:142-146 */
        return qmh_launch_attn_scores(m->d_q, kl, m->d_att, pos_ptr, c->n_heads, c->n_kv_heads, m->hd, S_,
                                      1.0f / sqrtf((float)m->hd), s);
    case ST_PV: /* src/model.c:147-154 */
        return qmh_launch_attn_pv(m->d_att, vl, m->d_xb, pos_ptr, c->n_heads, c->n_kv_heads, m->hd, S_, s);
    case ST_ATTN: /* src/model.c:137-156 in one launch */
        if (m->af_inst >= m->af_n) return (int)hipErrorNotSupported;
        return qmh_launch_attn_fused(m->d_q, kl, vl, m->d_xb, m->d_attp, pos_ptr, m->d_sync, c->n_heads, c->n_kv_heads,
                                     m->hd, S_, 1.0f / sqrtf((float)m->hd), l, c->n_layers, m->af_inst, m->af_cw,
                                     m->af_stall, s);
    case ST_WO: /* x += Wo xb (src/model.c:178-179) */
        mv_args_for(&L->wo, &a);
        a.x = m->d_xb;
        a.epi = QMH_EPI_ADD;
        a.out0 = m->d_x;
        return mv_launch(&a, s);
    case ST_W13: /* hb = silu(W1 rmsnorm(x)) * (W3 rmsnorm(x)) (src/model.c:181-184) */
        mv_args_for(&L->w13, &a);
        a.x = m->d_x;
        a.norm_w = m->d_norms + (size_t)(2 * l + 1) * D;
        a.eps = c->norm_eps;
        a.out0 = m->d_hb;
        if (L->w13.dtype == QMH_F32) {
            a.epi = QMH_EPI_STORE;
            int rc = mv_launch(&a, s);
            return rc ? rc : qmh_launch_swiglu(m->d_hb, m->d_hb + H, H, s);
        }
        a.epi = QMH_EPI_SWIGLU;
        if (L->w2_image) { /* hb goes straight to W2's quantized input (src/ops.c:59 on hb) */
            a.epi = QMH_EPI_SWIGLU_Q;
            a.out0 = NULL;
            a.xq_img = m->d_hq;
            a.xq_nb = (H + 31) / 32;
            a.xq_split = L->w2.dtype == QMH_Q4_0;
        }
        return mv_launch(&a, s);
    case ST_W2: /* x += W2 hb (src/model.c:185-186) */
        mv_args_for(&L->w2, &a);
        a.x = m->d_hb;
        if (L->w2_image) {
            a.x = NULL;
            a.xq_in = m->d_hq;
        }
        a.epi = QMH_EPI_ADD;
        a.out0 = m->d_x;
        return mv_launch(&a, s);
    case ST_OUT: /* logits = Woutput rmsnorm(x) (src/model.c:188-189) */
        mv_args_for(&m->output, &a);
        a.x = m->d_x;
        a.norm_w = m->d_norms + (size_t)(2 * c->n_layers) * D;
        a.eps = c->norm_eps;
        a.epi = QMH_EPI_STORE;
        a.out0 = m->d_logits;
        return mv_launch(&a, s);
    }
    return (int)hipErrorInvalidValue;
}

/* af: 0, or the attention in one launch by instance af - 1 (the step's position is below
 * qmh_attn_fused_max_n(af - 1)) */
static int enqueue_step(qmh_model *m, hipStream_t s, int with_argmax, int af) {
    const qmh_config *c = &m->cfg;
    if (af) m->af_inst = af - 1;
    LCHK(qmh_launch_embed(m->d_embd, m->emb_dtype, c->dim, c->vocab_size, m->d_tokpos, m->d_x, m->d_sync, s));
    static const int order[6] = {ST_QKV, ST_SCORES, ST_PV, ST_WO, ST_W13, ST_W2};
    static const int order_af[5] = {ST_QKV, ST_ATTN, ST_WO, ST_W13, ST_W2};
    for (int l = 0; l < c->n_layers; l++) {
        if (af)
            for (int k = 0; k < 5; k++) LCHK(enqueue_stage(m, order_af[k], l, s));
        else
            for (int k = 0; k < 6; k++) LCHK(enqueue_stage(m, order[k], l, s));
    }
    LCHK(enqueue_stage(m, ST_OUT, 0, s));
    if (with_argmax)
        LCHK(qmh_launch_argmax(m->d_logits, c->vocab_size, NULL, m->d_tokpos, m->d_record, c->max_seq, s));
    return 0;
}

/* the attention of a step at position pos: 0 (two launches) or 1 + the one-launch instance */
static int af_for(const qmh_model *m, int32_t pos) {
    for (int i = 0; i < m->af_n; i++)
        if (pos < qmh_attn_fused_max_n(i)) return i + 1;
    return 0;
}

/* one decode step at position pos on the library stream: a graph replay, or the same launches one by
 * one */
static hipError_t run_step(qmh_model *m, int with_argmax, int32_t pos) {
    const int af = af_for(m, pos);
    if (m->use_graph) {
        if (af) return hipGraphLaunch(with_argmax ? m->exec_greedy_af[af - 1] : m->exec_fwd_af[af - 1], g_stream);
        return hipGraphLaunch(with_argmax ? m->exec_greedy : m->exec_fwd, g_stream);
    }
    return enqueue_step(m, g_stream, with_argmax, af) ? hipErrorLaunchFailure : hipSuccess;
}

/* after a synchronization: the status of k_attn_fused's bounded waits since the last check (and the
 * word cleared for the next). copied: the caller already copied d_sync[1] to h_sync before it
 * synchronized */
static int check_attn_sync_copied(qmh_model *m, int copied) {
    if (!m->af_n) return 0;
    if (!copied) HIPCHK(hipMemcpy(m->h_sync, m->d_sync + 1, sizeof(uint32_t), hipMemcpyDeviceToHost));
    if (*m->h_sync == 0) return 0;
    const uint32_t st = *m->h_sync;
    HIPCHK(hipMemset(m->d_sync + 1, 0, sizeof(uint32_t)));
    return fail(st == 2 ? "attention: one-launch kernel given a context past its limit"
                        : "attention: a workgroup's wait for its head's scores ran out");
}
static int check_attn_sync(qmh_model *m) { return check_attn_sync_copied(m, 0); }

/* weight bytes one launch of a stage streams (the algorithmic bytes of the matvecs) */
static double stage_weight_bytes(const qmh_model *m, int which) {
    const struct qmh_weight *w = which == ST_QKV ? &m->layers[0].qkv
                                 : which == ST_WO ? &m->layers[0].wo
                                 : which == ST_W13 ? &m->layers[0].w13
                                 : which == ST_W2 ? &m->layers[0].w2
                                 : which == ST_OUT ? &m->output
                                                   : NULL;
    if (!w) return 0.0;
    const double rows = which == ST_W13 ? 2.0 * (double)w->rows : (double)w->rows;
    return rows * (double)qlm_row_bytes(w->dtype, w->cols);
}

int qmh_model_time_stage(qmh_model *m, int which, int32_t pos, int iters, double *ms_per_launch,
                         double *bytes_per_launch) {
    if (!m || which < 0 || which >= ST_COUNT || iters < 1 || pos < 0 || pos >= m->cfg.max_seq)
        return fail("time_stage: bad arguments");
    if (which == ST_ATTN) {
        const int af = af_for(m, pos);
        if (!af) return fail("time_stage: no one-launch attention for position %d", (int)pos);
        m->af_inst = af - 1;
    }
    /* the stages read token and position from device memory: set both (a greedy run leaves
     * the position one past its last step) */
    int32_t *slot = m->h_tokpos;
    slot[0] = 0, slot[1] = pos;
    HIPCHK(hipMemcpyAsync(m->d_tokpos, slot, sizeof(int32_t) * 2, hipMemcpyHostToDevice, g_stream));
    hipEvent_t e0, e1;
    HIPCHK(hipEventCreate(&e0));
    HIPCHK(hipEventCreate(&e1));
    int rc = 0;
    hipError_t e = hipEventRecord(e0, g_stream);
    for (int i = 0; i < iters && e == hipSuccess && rc == 0; i++)
        rc = enqueue_stage(m, which, which == ST_OUT ? 0 : i % m->cfg.n_layers, g_stream);
    if (e == hipSuccess && rc == 0) e = hipEventRecord(e1, g_stream);
    if (e == hipSuccess && rc == 0) e = hipEventSynchronize(e1);
    float ms = 0.0f;
    if (e == hipSuccess && rc == 0) e = hipEventElapsedTime(&ms, e0, e1);
    hipEventDestroy(e0);
    hipEventDestroy(e1);
    if (rc) return fail("time_stage launch: %s", hipGetErrorString((hipError_t)rc));
    if (e != hipSuccess) return fail("time_stage: %s", hipGetErrorString(e));
    if (ms_per_launch) *ms_per_launch = (double)ms / iters;
    if (bytes_per_launch) *bytes_per_launch = stage_weight_bytes(m, which);
    return 0;
}

/* HIP events around `iters` calls of body(i) on the library stream: ms per call */
static int time_calls(int iters, int (*body)(void *, int), void *ctx, double *ms_per_call, const char *what) {
    hipEvent_t e0, e1;
    HIPCHK(hipEventCreate(&e0));
    HIPCHK(hipEventCreate(&e1));
    int rc = 0;
    hipError_t e = hipEventRecord(e0, g_stream);
    for (int i = 0; i < iters && e == hipSuccess && rc == 0; i++) rc = body(ctx, i);
    if (e == hipSuccess && rc == 0) e = hipEventRecord(e1, g_stream);
    if (e == hipSuccess && rc == 0) e = hipEventSynchronize(e1);
    float ms = 0.0f;
    if (e == hipSuccess && rc == 0) e = hipEventElapsedTime(&ms, e0, e1);
    hipEventDestroy(e0);
    hipEventDestroy(e1);
    if (rc) return fail("%s launch: %s", what, hipGetErrorString((hipError_t)rc));
    if (e != hipSuccess) return fail("%s: %s", what, hipGetErrorString(e));
    if (ms_per_call) *ms_per_call = (double)ms / iters;
    return 0;
}

struct mv_time_ctx {
    const qmh_weight *const *w;
    int nw;
    const float *x;
    float *y;
};
static int mv_time_body(void *p, int i) {
    const struct mv_time_ctx *c = p;
    qmh_mv_args a;
    mv_args_for(c->w[i % c->nw], &a);
    a.x = c->x;
    a.epi = QMH_EPI_STORE;
    a.out0 = c->y;
    return mv_launch(&a, g_stream);
}

int qmh_time_matvec(const qmh_weight *const *W, int nw, const float *x, float *y, int iters, double *ms_per_call) {
    if (ensure()) return -1;
    if (!W || nw < 1 || !x || !y || iters < 1) return fail("time_matvec: bad arguments");
    for (int i = 0; i < nw; i++)
        if (!W[i] || W[i]->dtype != W[0]->dtype || W[i]->rows != W[0]->rows || W[i]->cols != W[0]->cols)
            return fail("time_matvec: the weights must share dtype and shape");
    struct mv_time_ctx c = {W, nw, x, y};
    return time_calls(iters, mv_time_body, &c, ms_per_call, "time_matvec");
}

struct mm_time_ctx {
    const float *A, *B;
    float *C;
    int64_t M, N, K;
};
static int mm_time_body(void *p, int i) {
    (void)i;
    const struct mm_time_ctx *c = p;
    return qmh_launch_gemm_nt(c->A, c->B, c->C, c->M, c->N, c->K, g_stream);
}

int qmh_time_matmul_nt(const float *A, const float *B, float *C, int64_t M, int64_t N, int64_t K, int iters,
                       double *ms_per_call) {
    if (ensure()) return -1;
    if (!A || !B || !C || M < 1 || N < 1 || K < 1 || iters < 1) return fail("time_matmul_nt: bad arguments");
    struct mm_time_ctx c = {A, B, C, M, N, K};
    return time_calls(iters, mm_time_body, &c, ms_per_call, "time_matmul_nt");
}

int qmh_model_time_greedy(qmh_model *m, int32_t token, int32_t pos, int32_t n_steps, int32_t *out, double *ms) {
    if (!m || n_steps < 1 || token < 0 || token >= m->cfg.vocab_size || pos < 0 ||
        (int64_t)pos + n_steps > m->cfg.max_seq)
        return fail("time_greedy: bad token/range");
    hipEvent_t e0, e1;
    HIPCHK(hipEventCreate(&e0));
    HIPCHK(hipEventCreate(&e1));
    int32_t *slot = m->h_tokpos;
    slot[0] = token, slot[1] = pos, slot[2] = 0, slot[3] = 0;
    hipError_t e = hipMemcpyAsync(m->d_tokpos, slot, sizeof(int32_t) * 4, hipMemcpyHostToDevice, g_stream);
    if (e == hipSuccess) e = hipEventRecord(e0, g_stream);
    for (int32_t k = 0; k < n_steps && e == hipSuccess; k++) e = run_step(m, 1, pos + k);
    if (e == hipSuccess) e = hipEventRecord(e1, g_stream);
    if (e == hipSuccess && out)
        e = hipMemcpyAsync(out, m->d_record, sizeof(int32_t) * (size_t)n_steps, hipMemcpyDeviceToHost, g_stream);
    if (e == hipSuccess) e = hipStreamSynchronize(g_stream);
    float t = 0.0f;
    if (e == hipSuccess) e = hipEventElapsedTime(&t, e0, e1);
    hipEventDestroy(e0);
    hipEventDestroy(e1);
    if (e != hipSuccess) return fail("time_greedy: %s", hipGetErrorString(e));
    if (ms) *ms = (double)t;
    return check_attn_sync(m);
}

static int capture(qmh_model *m, int with_argmax, int af, hipGraph_t *g, hipGraphExec_t *ex) {
    HIPCHK(hipStreamBeginCapture(g_stream, hipStreamCaptureModeThreadLocal));
    int rc = enqueue_step(m, g_stream, with_argmax, af);
    hipGraph_t graph = NULL;
    hipError_t e = hipStreamEndCapture(g_stream, &graph);
    if (rc) {
        if (graph) hipGraphDestroy(graph);
        return rc;
    }
    if (e != hipSuccess) return fail("graph capture: %s", hipGetErrorString(e));
    e = hipGraphInstantiate(ex, graph, NULL, NULL, 0);
    if (e != hipSuccess) {
        hipGraphDestroy(graph);
        return fail("graph instantiate: %s", hipGetErrorString(e));
    }
    *g = graph;
    return 0;
}

void qmh_model_free(qmh_model *m) {
    if (!m) return;
    if (g_ready) hipStreamSynchronize(g_stream);
    if (m->exec_fwd) hipGraphExecDestroy(m->exec_fwd);
    if (m->exec_greedy) hipGraphExecDestroy(m->exec_greedy);
    if (m->graph_fwd) hipGraphDestroy(m->graph_fwd);
    if (m->graph_greedy) hipGraphDestroy(m->graph_greedy);
    for (int i = 0; i < 2; i++) {
        if (m->exec_fwd_af[i]) hipGraphExecDestroy(m->exec_fwd_af[i]);
        if (m->exec_greedy_af[i]) hipGraphExecDestroy(m->exec_greedy_af[i]);
        if (m->graph_fwd_af[i]) hipGraphDestroy(m->graph_fwd_af[i]);
        if (m->graph_greedy_af[i]) hipGraphDestroy(m->graph_greedy_af[i]);
    }
    if (m->layers) {
        for (int l = 0; l < m->cfg.n_layers; l++) {
            weight_release(&m->layers[l].qkv);
            weight_release(&m->layers[l].wo);
            weight_release(&m->layers[l].w13);
            weight_release(&m->layers[l].w2);
        }
        free(m->layers);
    }
    weight_release(&m->output);
    void *dev[] = {m->d_embd,   m->d_norms,  m->d_rope,     m->d_x,    m->d_xb,   m->d_q,     m->d_hb,
                   m->d_hq,     m->d_att,    m->d_logits,   m->d_kt,   m->d_v,    m->d_tokpos, m->d_record,
                   m->d_pf_tok, m->d_pf_x,   m->d_pf_xb,    m->d_pf_q, m->d_pf_hb, m->d_pf_att, m->d_pf_logits,
                   m->d_pf_xd,  m->d_pf_xc,  m->d_pf_xc2, m->d_pf_xd2, m->d_attp, m->d_sync};
    for (size_t i = 0; i < sizeof dev / sizeof dev[0]; i++)
        if (dev[i]) hipFree(dev[i]);
    if (m->h_tokpos) hipHostFree(m->h_tokpos);
    if (m->h_sync) hipHostFree(m->h_sync);
    if (m->h_logits) hipHostFree(m->h_logits);
    if (m->h_pf_tok) hipHostFree(m->h_pf_tok);
    free(m);
}

static int check_view(const qmh_tensor_view *t, const char *name, int64_t d0, int64_t d1) {
    int ok = t && t->data &&
             ((d1 == 0 && t->ndim == 1 && t->ne[0] == d0 && t->dtype == QMH_F32) ||
              (d1 != 0 && t->ndim == 2 && t->ne[0] == d0 && t->ne[1] == d1 &&
               (t->dtype == QMH_F32 || t->dtype == QMH_Q8_0 || t->dtype == QMH_Q4_0)));
    return ok ? 0 : fail("missing or mis-shaped tensor '%s'", name);
}

static int model_build(qmh_model *m, const qmh_tensor_view *tok_embd, const qmh_tensor_view *norm,
                       const qmh_tensor_view *output, const qmh_tensor_view *layers) {
    const qmh_config *c = &m->cfg;
    if (c->dim <= 0 || c->hidden_dim <= 0 || c->n_layers <= 0 || c->n_heads <= 0 || c->n_kv_heads <= 0 ||
        c->vocab_size <= 0 || c->max_seq <= 0)
        return fail("invalid config");
    /* reference src/model.c:48-52 */
    if (c->dim % c->n_heads || c->n_heads % c->n_kv_heads || (c->dim / c->n_heads) % 2 || c->n_layers > 1024)
        return fail("inconsistent head configuration");
    const int64_t D = c->dim, H = c->hidden_dim, V = c->vocab_size, S_ = c->max_seq;
    m->hd = c->dim / c->n_heads;
    m->kvd = m->hd * c->n_kv_heads;
    m->group = c->n_heads / c->n_kv_heads;
    const int64_t KV = m->kvd;
    if (check_view(tok_embd, "tok_embd", V, D) || check_view(norm, "norm", D, 0) || check_view(output, "output", V, D))
        return -1;
    static const char *sfx[9] = {"attn_norm", "wq", "wk", "wv", "wo", "ffn_norm", "w1", "w2", "w3"};
    const int64_t shp[9][2] = {{D, 0}, {D, D}, {KV, D}, {KV, D}, {D, D}, {D, 0}, {H, D}, {D, H}, {H, D}};
    for (int l = 0; l < c->n_layers; l++)
        for (int k = 0; k < 9; k++) {
            char nm[64];
            snprintf(nm, sizeof nm, "layers.%d.%s", l, sfx[k]);
            if (check_view(&layers[9 * l + k], nm, shp[k][0], shp[k][1])) return -1;
        }
    for (int l = 0; l < c->n_layers; l++) {
        const qmh_tensor_view *t = &layers[9 * l];
        if (t[1].dtype != t[2].dtype || t[1].dtype != t[3].dtype)
            return fail("layer %d: wq/wk/wv must share one dtype", l);
        if (t[6].dtype != t[8].dtype) return fail("layer %d: w1/w3 must share one dtype", l);
    }
    /* LDS budget of the kernels (64 KiB per workgroup); W2's input is the quantized image W1|W3 writes
     * when both are quantized (every layer), else hb quantized in W2's prologue */
    int h_image = 1;
    for (int l = 0; l < c->n_layers; l++)
        if (layers[9 * l + 6].dtype == QMH_F32 || layers[9 * l + 7].dtype == QMH_F32) h_image = 0;
    const int hmax = h_image && qmh_matvec_max_image_cols() > qmh_matvec_max_cols(0) ? qmh_matvec_max_image_cols()
                                                                                      : qmh_matvec_max_cols(0);
    const int nbD = (int)((D + 31) / 32), nbH = (int)((H + 31) / 32);
    if (qmh_matvec_grid(1, nbD, 64, QMH_Q4_0, 1) < 1 || qmh_matvec_grid(1, nbD, QMH_TILE_R, QMH_Q4_0, 1) < 1 ||
        qmh_matvec_grid(1, nbD, 8, QMH_Q4_0, 1) < 1 || qmh_matvec_grid(1, nbH, 8, QMH_Q4_0, 1) < 1 ||
        D > qmh_matvec_max_cols(1) || H > hmax)
        return fail("model dims exceed the kernels' limits (dim <= %d, hidden_dim <= %d)", qmh_matvec_max_cols(1),
                    hmax);
    /* any group (the reference's only rule is n_heads % n_kv_heads == 0): the kv-head P.V kernel takes
     * it in sub-groups of up to 16 query heads */
    const int64_t gsub = m->group < 16 ? m->group : 16;
    if (((int64_t)64 * (m->hd + 1) + gsub * m->hd) * 4 > 65536)
        return fail("head_dim too large for the attention kernels");

    HIPCHK(hipMalloc(&m->d_embd, (size_t)V * qlm_row_bytes(tok_embd->dtype, D)));
    HIPCHK(hipMemcpy(m->d_embd, tok_embd->data, (size_t)V * qlm_row_bytes(tok_embd->dtype, D), hipMemcpyHostToDevice));
    m->emb_dtype = tok_embd->dtype;
    HIPCHK(hipMalloc((void **)&m->d_norms, sizeof(float) * (size_t)(2 * c->n_layers + 1) * D));
    m->layers = calloc((size_t)c->n_layers, sizeof(dev_layer));
    if (!m->layers) return fail("out of memory");
    for (int l = 0; l < c->n_layers; l++) {
        const qmh_tensor_view *t = &layers[9 * l];
        HIPCHK(hipMemcpy(m->d_norms + (size_t)(2 * l) * D, t[0].data, sizeof(float) * D, hipMemcpyHostToDevice));
        HIPCHK(hipMemcpy(m->d_norms + (size_t)(2 * l + 1) * D, t[5].data, sizeof(float) * D, hipMemcpyHostToDevice));
        dev_layer *L = &m->layers[l];
        const void *qkv[3] = {t[1].data, t[2].data, t[3].data};
        const int64_t qkv_rows[3] = {D, KV, KV};
        if (weight_build(&L->qkv, t[1].dtype, 3, qkv, qkv_rows, D, 0, QMH_TILE_R)) return -1;
        const void *wo[1] = {t[4].data};
        const int64_t wo_rows[1] = {D};
        if (weight_build(&L->wo, t[4].dtype, 1, wo, wo_rows, D, 0, 8)) return -1;
        const void *w13[2] = {t[6].data, t[8].data};
        const int64_t w13_rows[2] = {H, H};
        L->w2_image = t[6].dtype != QMH_F32 && t[7].dtype != QMH_F32;
        if (weight_build(&L->w13, t[6].dtype, 2, w13, w13_rows, D, t[6].dtype != QMH_F32, L->w2_image ? 64 : 32))
            return -1;
        const void *w2[1] = {t[7].data};
        const int64_t w2_rows[1] = {D};
        if (weight_build(&L->w2, t[7].dtype, 1, w2, w2_rows, H, 0, 8)) return -1;
    }
    HIPCHK(hipMemcpy(m->d_norms + (size_t)(2 * c->n_layers) * D, norm->data, sizeof(float) * D, hipMemcpyHostToDevice));
    const void *out[1] = {output->data};
    const int64_t out_rows[1] = {V};
    if (weight_build(&m->output, output->dtype, 1, out, out_rows, D, 0, QMH_TILE_R)) return -1;

    /* RoPE table for every position, reference formula (src/ops.c:114-126) */
    const size_t pairs = (size_t)S_ * (size_t)(m->hd / 2);
    float *tab = malloc(sizeof(float) * 2 * (pairs ? pairs : 1));
    if (!tab) return fail("out of memory");
    for (int64_t p = 0; p < S_; p++) rope_pairs(tab + (size_t)p * m->hd, m->hd, p, c->rope_theta);
    hipError_t e = hipMalloc((void **)&m->d_rope, sizeof(float) * 2 * (pairs ? pairs : 1));
    if (e == hipSuccess) e = hipMemcpy(m->d_rope, tab, sizeof(float) * 2 * pairs, hipMemcpyHostToDevice);
    free(tab);
    if (e != hipSuccess) return fail("rope table: %s", hipGetErrorString(e));

    /* activations and caches (zeroed like the reference's arena, src/arena.c:6-15) */
    g_exact_norm = getenv("QMH_EXACT_NORM") != NULL;
    const size_t kv_bytes = sizeof(float) * (size_t)c->n_layers * (size_t)S_ * (size_t)KV;
    HIPCHK(hipMalloc((void **)&m->d_x, sizeof(float) * D));
    HIPCHK(hipMalloc((void **)&m->d_xb, sizeof(float) * D));
    HIPCHK(hipMalloc((void **)&m->d_q, sizeof(float) * D));
    HIPCHK(hipMalloc((void **)&m->d_hb, sizeof(float) * 2 * H));
    HIPCHK(hipMemsetAsync(m->d_x, 0, sizeof(float) * D, g_stream));
    HIPCHK(hipMemsetAsync(m->d_xb, 0, sizeof(float) * D, g_stream));
    HIPCHK(hipMemsetAsync(m->d_q, 0, sizeof(float) * D, g_stream));
    HIPCHK(hipMemsetAsync(m->d_hb, 0, sizeof(float) * 2 * H, g_stream));
    HIPCHK(hipMalloc(&m->d_hq, QMH_XQ_IMAGE_BYTES((H + 31) / 32)));
    HIPCHK(hipMemsetAsync(m->d_hq, 0, QMH_XQ_IMAGE_BYTES((H + 31) / 32), g_stream)); /* the pad reads as 0 */
    HIPCHK(hipMalloc((void **)&m->d_att, sizeof(float) * (size_t)c->n_heads * S_));
    HIPCHK(hipMalloc((void **)&m->d_logits, sizeof(float) * V));
    HIPCHK(hipMalloc((void **)&m->d_kt, kv_bytes));
    HIPCHK(hipMalloc((void **)&m->d_v, kv_bytes));
    HIPCHK(hipMalloc((void **)&m->d_tokpos, sizeof(int32_t) * 4));
    HIPCHK(hipMalloc((void **)&m->d_record, sizeof(int32_t) * (size_t)S_));
    HIPCHK(hipMemsetAsync(m->d_kt, 0, kv_bytes, g_stream));
    HIPCHK(hipMemsetAsync(m->d_v, 0, kv_bytes, g_stream));
    HIPCHK(hipMemsetAsync(m->d_tokpos, 0, sizeof(int32_t) * 4, g_stream));
    /* the one-launch attention: its score words start at epoch 0, which no launch uses */
    {
        /* QMH_AF_CW=16 or 8 (tests): the column width instead of the one chosen for the shape */
        const char *cw = getenv("QMH_AF_CW");
        m->af_cw = cw && (atoi(cw) == 16 || atoi(cw) == 8) ? atoi(cw) : qmh_attn_fused_cw(c->n_heads, m->hd);
    }
    m->af_n = getenv("QMH_NO_FUSED_ATTN") ? 0
                                          : qmh_attn_fused_supported(c->n_heads, c->n_kv_heads, m->hd, (int)S_, m->af_cw);
    if (m->af_n > 1 && getenv("QMH_FUSED_ATTN_640")) m->af_n = 1;
    m->af_stall = getenv("QMH_AF_FORCE_STALL") != NULL;
    HIPCHK(hipMalloc((void **)&m->d_sync, sizeof(uint32_t) * 2));
    HIPCHK(hipMemsetAsync(m->d_sync, 0, sizeof(uint32_t) * 2, g_stream));
    HIPCHK(hipHostMalloc((void **)&m->h_sync, sizeof(uint32_t), hipHostMallocDefault));
    if (m->af_n) {
        HIPCHK(hipMalloc((void **)&m->d_attp, sizeof(uint64_t) * (size_t)c->n_heads * S_));
        HIPCHK(hipMemsetAsync(m->d_attp, 0, sizeof(uint64_t) * (size_t)c->n_heads * S_, g_stream));
    }
    HIPCHK(hipHostMalloc((void **)&m->h_tokpos, sizeof(int32_t) * 4 * (size_t)S_, hipHostMallocDefault));
    HIPCHK(hipHostMalloc((void **)&m->h_logits, sizeof(float) * V, hipHostMallocDefault));
    /* batched prefill buffers (models whose matrices are all quantized) */
    /* the batched prompt path's attention (k_pf_*, k_bt_*) takes head_dim <= 128 in whole float4s;
     * other models run the prompt as sequential forwards */
    m->pf_ok = m->output.dtype != QMH_F32 && m->hd <= 128 && m->hd % 4 == 0;
    for (int l = 0; l < c->n_layers && m->pf_ok; l++) {
        const dev_layer *L = &m->layers[l];
        m->pf_ok = L->qkv.dtype != QMH_F32 && L->wo.dtype != QMH_F32 && L->w13.dtype != QMH_F32 &&
                   L->w2.dtype != QMH_F32;
    }
    if (m->pf_ok) {
        m->pf_cap = S_ < 512 ? (int)S_ : 512;
        m->pf_pp = (m->pf_cap + 127) / 128 * 128;
        const size_t PP = (size_t)m->pf_pp, nbmax = (size_t)((D > H ? D : H) + 31) / 32;
        HIPCHK(hipMalloc((void **)&m->d_pf_tok, sizeof(int32_t) * PP));
        HIPCHK(hipHostMalloc((void **)&m->h_pf_tok, sizeof(int32_t) * PP, hipHostMallocDefault));
        HIPCHK(hipMalloc((void **)&m->d_pf_x, sizeof(float) * PP * D));
        HIPCHK(hipMalloc((void **)&m->d_pf_xb, sizeof(float) * PP * D));
        HIPCHK(hipMalloc((void **)&m->d_pf_q, sizeof(float) * PP * D));
        HIPCHK(hipMalloc((void **)&m->d_pf_hb, sizeof(float) * PP * H));
        HIPCHK(hipMalloc((void **)&m->d_pf_att, sizeof(float) * (size_t)c->n_heads * PP * S_));
        HIPCHK(hipMalloc((void **)&m->d_pf_logits, sizeof(float) * PP * V));
        HIPCHK(hipMalloc((void **)&m->d_pf_xc, 32 * nbmax * PP));
        HIPCHK(hipMalloc((void **)&m->d_pf_xd, sizeof(float) * nbmax * PP));
        HIPCHK(hipMalloc((void **)&m->d_pf_xc2, 32 * nbmax * PP));
        HIPCHK(hipMalloc((void **)&m->d_pf_xd2, sizeof(float) * nbmax * PP));
        /* padding tokens of the images feed the MFMAs columns whose results are never stored: zeroed
         * once so that they hold finite values */
        HIPCHK(hipMemsetAsync(m->d_pf_xc, 0, 32 * nbmax * PP, g_stream));
        HIPCHK(hipMemsetAsync(m->d_pf_xd, 0, sizeof(float) * nbmax * PP, g_stream));
        HIPCHK(hipMemsetAsync(m->d_pf_xc2, 0, 32 * nbmax * PP, g_stream));
        HIPCHK(hipMemsetAsync(m->d_pf_xd2, 0, sizeof(float) * nbmax * PP, g_stream));
    }
    HIPCHK(hipStreamSynchronize(g_stream));
    m->use_graph = getenv("QMH_NO_GRAPH") == NULL;
    if (m->use_graph && capture(m, 0, 0, &m->graph_fwd, &m->exec_fwd)) return -1;
    if (m->use_graph && capture(m, 1, 0, &m->graph_greedy, &m->exec_greedy)) return -1;
    for (int i = 0; i < m->af_n; i++) {
        if (m->use_graph && capture(m, 0, i + 1, &m->graph_fwd_af[i], &m->exec_fwd_af[i])) return -1;
        if (m->use_graph && capture(m, 1, i + 1, &m->graph_greedy_af[i], &m->exec_greedy_af[i])) return -1;
    }
    if (!m->use_graph && enqueue_step(m, g_stream, 0, 0)) return -1; /* validate the launches once */
    for (int i = 0; i < m->af_n; i++)
        if (!m->use_graph && enqueue_step(m, g_stream, 0, i + 1)) return -1;
    HIPCHK(hipStreamSynchronize(g_stream));
    return 0;
}

qmh_model *qmh_model_create(const qmh_config *cfg, const qmh_tensor_view *tok_embd, const qmh_tensor_view *norm,
                            const qmh_tensor_view *output, const qmh_tensor_view *layers) {
    if (ensure()) return NULL;
    if (!cfg || !tok_embd || !norm || !output || !layers) {
        fail("model_create: NULL argument");
        return NULL;
    }
    qmh_model *m = calloc(1, sizeof *m);
    if (!m) {
        fail("out of memory");
        return NULL;
    }
    m->cfg = *cfg;
    if (model_build(m, tok_embd, norm, output, layers)) {
        char keep[sizeof g_err];
        memcpy(keep, g_err, sizeof keep);
        qmh_model_free(m);
        memcpy(g_err, keep, sizeof keep);
        return NULL;
    }
    return m;
}

qmh_model *qmh_model_load(const char *path, int32_t max_seq) {
    if (ensure()) return NULL;
    qlm_map f;
    char err[256];
    if (qlm_map_open(&f, path, err, sizeof err)) {
        fail("%s", err);
        return NULL;
    }
    static const char *keys[7] = {"llama.dim",        "llama.hidden_dim", "llama.n_layers", "llama.n_heads",
                                  "llama.n_kv_heads", "llama.vocab_size", "llama.max_seq"};
    for (int k = 0; k < 7; k++)
        if (!f.have[k]) { /* reference src/model.c:9-16 */
            fail("missing/invalid metadata '%s'", keys[k]);
            qlm_map_close(&f);
            return NULL;
        }
    qmh_config cfg = f.cfg;
    if (max_seq > 0 && max_seq < cfg.max_seq) cfg.max_seq = max_seq;
    const qlm_tensor *te = qlm_map_find(&f, "tok_embd"), *tn = qlm_map_find(&f, "norm"),
                     *to = qlm_map_find(&f, "output");
    qmh_tensor_view *lv = calloc((size_t)(cfg.n_layers > 0 ? cfg.n_layers : 1) * 9, sizeof(qmh_tensor_view));
    qmh_model *m = NULL;
    if (!te || !tn || !to || !lv) {
        fail("missing or mis-shaped tensor '%s'", !te ? "tok_embd" : !tn ? "norm" : "output");
        goto done;
    }
    static const char *sfx[9] = {"attn_norm", "wq", "wk", "wv", "wo", "ffn_norm", "w1", "w2", "w3"};
    for (int l = 0; l < cfg.n_layers && l <= 1024; l++)
        for (int k = 0; k < 9; k++) {
            char nm[64];
            snprintf(nm, sizeof nm, "layers.%d.%s", l, sfx[k]);
            const qlm_tensor *t = qlm_map_find(&f, nm);
            if (!t) {
                fail("missing or mis-shaped tensor '%s'", nm);
                goto done;
            }
            lv[9 * l + k] = t->view;
        }
    m = qmh_model_create(&cfg, &te->view, &tn->view, &to->view, lv);
done:
    free(lv);
    qlm_map_close(&f);
    return m;
}

const qmh_config *qmh_model_config(const qmh_model *m) { return m ? &m->cfg : NULL; }

int qmh_qlm_config(const char *path, int32_t max_seq, qmh_config *out) {
    if (!path || !out) return fail("qlm_config: NULL argument");
    qlm_map f;
    char err[256];
    if (qlm_map_open(&f, path, err, sizeof err)) return fail("%s", err);
    static const char *keys[7] = {"llama.dim",        "llama.hidden_dim", "llama.n_layers", "llama.n_heads",
                                  "llama.n_kv_heads", "llama.vocab_size", "llama.max_seq"};
    qmh_config c = f.cfg;
    int rc = 0;
    for (int k = 0; k < 7 && rc == 0; k++)
        if (!f.have[k]) rc = fail("missing/invalid metadata '%s'", keys[k]); /* src/model.c:8-16 */
    if (rc == 0 && (c.dim % c.n_heads || c.n_heads % c.n_kv_heads || (c.dim / c.n_heads) % 2 || c.n_layers > 1024))
        rc = fail("inconsistent head configuration"); /* src/model.c:48-52 */
    if (rc == 0 && max_seq > 0 && max_seq < c.max_seq) c.max_seq = max_seq; /* src/model.c:53 */
    qlm_map_close(&f);
    if (rc == 0) *out = c;
    return rc;
}

float *qmh_model_forward(qmh_model *m, int32_t token, int32_t pos) {
    if (!m || token < 0 || token >= m->cfg.vocab_size || pos < 0 || pos >= m->cfg.max_seq) return NULL;
    m->h_tokpos[0] = token;
    m->h_tokpos[1] = pos;
    hipError_t e = hipMemcpyAsync(m->d_tokpos, m->h_tokpos, sizeof(int32_t) * 2, hipMemcpyHostToDevice, g_stream);
    if (e == hipSuccess) e = run_step(m, 0, pos);
    if (e == hipSuccess)
        e = hipMemcpyAsync(m->h_logits, m->d_logits, sizeof(float) * (size_t)m->cfg.vocab_size, hipMemcpyDeviceToHost,
                           g_stream);
    if (e == hipSuccess && m->af_n)
        e = hipMemcpyAsync(m->h_sync, m->d_sync + 1, sizeof(uint32_t), hipMemcpyDeviceToHost, g_stream);
    if (e == hipSuccess) e = hipStreamSynchronize(g_stream);
    if (e != hipSuccess) {
        fail("forward: %s", hipGetErrorString(e));
        return NULL;
    }
    if (check_attn_sync_copied(m, 1)) return NULL;
    return m->h_logits;
}

/* the batched matmul over the prefill activation image (d_pf_xc/xd) with weight w */
static void pf_args_for(const qmh_model *m, const struct qmh_weight *w, int P, qmh_pf_args *a) {
    memset(a, 0, sizeof *a);
    a->dtype = w->dtype;
    a->codes = w->codes;
    a->scales = w->scales;
    a->nb = w->nb;
    a->tile_r = w->tile_r;
    a->rows = (int)w->rows;
    a->xc = m->d_pf_xc;
    a->xd = m->d_pf_xd;
    a->PP = m->pf_pp;
    a->P = P;
}

/* independent sequences of a batched decode step: token p at position pos[p] (device), its caches
 * at kt/v + p*kv_stride; max_pos is the largest position */
typedef struct {
    const int32_t *pos;
    int max_pos;
    float *kt, *v;
    long long kv_stride;
} pf_seqs;

/* one layer for P tokens (src/model.c:164-187, token by token in the reference): a prompt at positions
 * pos.. in the model's caches, or (bt != NULL) one token of each of P independent sequences */
static int pf_layer(qmh_model *m, int l, int P, int pos, const pf_seqs *bt, hipStream_t s) {
    const qmh_config *c = &m->cfg;
    const int D = c->dim, H = c->hidden_dim, S_ = c->max_seq;
    dev_layer *L = &m->layers[l];
    float *kl = m->d_kt + (size_t)l * S_ * m->kvd, *vl = m->d_v + (size_t)l * S_ * m->kvd;
    if (bt) {
        kl = bt->kt + (size_t)l * P * bt->kv_stride;
        vl = bt->v + (size_t)l * P * bt->kv_stride;
    }
    qmh_pf_args a;
    /* q, k, v = W rmsnorm(x); rope; k, v -> caches */
    pf_args_for(m, &L->qkv, P, &a);
    a.xf = m->d_pf_x;
    a.ldxf = D;
    a.nxf = D;
    a.norm_w = m->d_norms + (size_t)(2 * l) * D;
    a.eps = c->norm_eps;
    a.rows_alloc = L->qkv.ntiles * L->qkv.tile_r;
    a.epi = QMH_PF_QKV;
    a.out0 = m->d_pf_q;
    a.ld0 = D;
    a.out1 = kl;
    a.out2 = vl;
    a.seg1 = D;
    a.seg2 = D + m->kvd;
    a.rope = m->d_rope;
    a.pos0 = pos;
    a.head_dim = m->hd;
    a.max_seq = S_;
    a.kvd = m->kvd;
    if (bt) {
        a.pos_arr = bt->pos;
        a.kv_stride = bt->kv_stride;
    }
    LCHK(qmh_launch_pf_gemm(&a, s));
    if (bt)
        LCHK(qmh_launch_bt_attention(m->d_pf_q, kl, vl, bt->kv_stride, bt->pos, bt->max_pos, m->d_pf_att, m->d_pf_xb,
                                     P, c->n_heads, c->n_kv_heads, m->hd, S_, 1.0f / sqrtf((float)m->hd), 0, s));
    /* head_dim 128 or 64: P.V also writes xb as Wo's quantized input image */
    const int xb_image = !bt && (m->hd == 128 || m->hd == 64);
    if (!bt)
        LCHK(qmh_launch_pf_attention(m->d_pf_q, kl, vl, m->d_pf_att, m->d_pf_xb, P, pos, c->n_heads, c->n_kv_heads,
                                     m->hd, S_, 1.0f / sqrtf((float)m->hd), xb_image ? m->d_pf_xc : NULL,
                                     xb_image ? m->d_pf_xd : NULL, m->pf_pp, L->wo.dtype == QMH_Q4_0, s));
    /* x += Wo xb */
    pf_args_for(m, &L->wo, P, &a);
    a.xf = xb_image ? NULL : m->d_pf_xb;
    a.ldxf = D;
    a.nxf = D;
    a.norm_w = NULL;
    a.eps = 0.0f;
    a.rows_alloc = L->wo.ntiles * L->wo.tile_r;
    a.epi = QMH_PF_ADD;
    a.out0 = m->d_pf_x;
    a.ld0 = D;
    LCHK(qmh_launch_pf_gemm(&a, s));
    /* hb = silu(W1 rmsnorm(x)) * (W3 rmsnorm(x)) */
    pf_args_for(m, &L->w13, P, &a);
    a.xf = m->d_pf_x;
    a.ldxf = D;
    a.nxf = D;
    a.norm_w = m->d_norms + (size_t)(2 * l + 1) * D;
    a.eps = c->norm_eps;
    a.il = 1;
    a.rows_alloc = L->w13.ntiles * (L->w13.tile_r / 2);
    a.epi = QMH_PF_SWIGLU;
    a.out0 = m->d_pf_hb;
    a.ld0 = H;
    /* past the skinny matmul's token counts (the tiled matmul) hb is written only as W2's quantized
     * image */
    const int hb_image = P > QMH_PF_SKINNY_P;
    if (hb_image) {
        a.qxc = m->d_pf_xc2;
        a.qxd = m->d_pf_xd2;
        a.qperm8 = L->w2.dtype == QMH_Q4_0;
    }
    LCHK(qmh_launch_pf_gemm(&a, s));
    /* x += W2 hb */
    pf_args_for(m, &L->w2, P, &a);
    a.xf = hb_image ? NULL : m->d_pf_hb;
    if (hb_image) {
        a.xc = m->d_pf_xc2;
        a.xd = m->d_pf_xd2;
    }
    a.ldxf = H;
    a.nxf = H;
    a.norm_w = NULL;
    a.eps = 0.0f;
    a.rows_alloc = L->w2.ntiles * L->w2.tile_r;
    a.epi = QMH_PF_ADD;
    a.out0 = m->d_pf_x;
    a.ld0 = D;
    LCHK(qmh_launch_pf_gemm(&a, s));
    return 0;
}

/* the prompt in passes of up to pf_cap tokens. Logits (mode): none; the last position's; or every
 * position's (the reference's prompt loop computes them all), into d_pf_logits and, when host is given,
 * copied there (host[V] for the last, host[n*V] for all) */
enum { PF_LOGITS_NONE = 0, PF_LOGITS_LAST = 1, PF_LOGITS_ALL = 2 };
static int pf_batched(qmh_model *m, const int32_t *tokens, int32_t n, int32_t pos0, int mode, float *host) {
    const qmh_config *c = &m->cfg;
    const int D = c->dim, V = c->vocab_size;
    for (int32_t c0 = 0; c0 < n; c0 += m->pf_cap) {
        const int P = n - c0 < m->pf_cap ? n - c0 : m->pf_cap, pos = pos0 + c0;
        memcpy(m->h_pf_tok, tokens + c0, sizeof(int32_t) * (size_t)P);
        HIPCHK(hipMemcpyAsync(m->d_pf_tok, m->h_pf_tok, sizeof(int32_t) * (size_t)P, hipMemcpyHostToDevice, g_stream));
        LCHK(qmh_launch_pf_embed(m->d_embd, m->emb_dtype, D, V, m->d_pf_tok, P, m->d_pf_x, g_stream));
        for (int l = 0; l < c->n_layers; l++)
            if (pf_layer(m, l, P, pos, NULL, g_stream)) return -1;
        const int last = c0 + P == n;
        if (mode == PF_LOGITS_ALL || (mode == PF_LOGITS_LAST && last)) {
            /* logits = Woutput rmsnorm(x) (src/model.c:188-189): every position, or the last one */
            const int rows = mode == PF_LOGITS_ALL ? P : 1;
            qmh_pf_args a;
            pf_args_for(m, &m->output, rows, &a);
            a.xf = m->d_pf_x + (size_t)(P - rows) * D;
            a.ldxf = D;
            a.nxf = D;
            a.norm_w = m->d_norms + (size_t)(2 * c->n_layers) * D;
            a.eps = c->norm_eps;
            a.rows_alloc = m->output.ntiles * m->output.tile_r;
            a.epi = QMH_PF_STORE;
            a.out0 = m->d_pf_logits;
            a.ld0 = V;
            LCHK(qmh_launch_pf_gemm(&a, g_stream));
            if (host)
                HIPCHK(hipMemcpyAsync(host + (mode == PF_LOGITS_ALL ? (size_t)c0 * V : 0), m->d_pf_logits,
                                      sizeof(float) * (size_t)rows * V, hipMemcpyDeviceToHost, g_stream));
        }
        /* h_pf_tok is reused by the next pass; after the last one the caller synchronizes (the
           timed prefill records its end event first) */
        if (c0 + P < n) HIPCHK(hipStreamSynchronize(g_stream));
    }
    return 0;
}

int qmh_model_prefill(qmh_model *m, const int32_t *tokens, int32_t n, int32_t pos0, float *logits) {
    if (!m || !tokens || n < 0 || pos0 < 0 || (int64_t)pos0 + n > m->cfg.max_seq) return fail("prefill: bad range");
    for (int32_t i = 0; i < n; i++)
        if (tokens[i] < 0 || tokens[i] >= m->cfg.vocab_size) return fail("prefill: token %d out of range", tokens[i]);
    if (m->pf_ok && getenv("QMH_PREFILL_SEQ") == NULL) {
        if (pf_batched(m, tokens, n, pos0, logits ? PF_LOGITS_ALL : PF_LOGITS_NONE, logits)) return -1;
        HIPCHK(hipStreamSynchronize(g_stream));
        return 0;
    }
    const size_t V = (size_t)m->cfg.vocab_size;
    for (int32_t i = 0; i < n; i++) {
        int32_t *slot = m->h_tokpos + 4 * (size_t)i;
        slot[0] = tokens[i];
        slot[1] = pos0 + i;
        HIPCHK(hipMemcpyAsync(m->d_tokpos, slot, sizeof(int32_t) * 2, hipMemcpyHostToDevice, g_stream));
        HIPCHK(run_step(m, 0, pos0 + i));
        if (logits) HIPCHK(hipMemcpyAsync(logits + (size_t)i * V, m->d_logits, sizeof(float) * V, hipMemcpyDeviceToHost, g_stream));
    }
    HIPCHK(hipStreamSynchronize(g_stream));
    return check_attn_sync(m);
}

int qmh_model_greedy(qmh_model *m, int32_t token, int32_t pos, int32_t n_steps, int32_t *out) {
    if (!m || n_steps < 0 || token < 0 || token >= m->cfg.vocab_size || pos < 0 ||
        (int64_t)pos + n_steps > m->cfg.max_seq)
        return fail("greedy: bad token/range");
    int32_t *slot = m->h_tokpos;
    slot[0] = token, slot[1] = pos, slot[2] = 0, slot[3] = 0;
    HIPCHK(hipMemcpyAsync(m->d_tokpos, slot, sizeof(int32_t) * 4, hipMemcpyHostToDevice, g_stream));
    for (int32_t k = 0; k < n_steps; k++) HIPCHK(run_step(m, 1, pos + k));
    if (n_steps > 0 && out)
        HIPCHK(hipMemcpyAsync(out, m->d_record, sizeof(int32_t) * (size_t)n_steps, hipMemcpyDeviceToHost, g_stream));
    HIPCHK(hipStreamSynchronize(g_stream));
    return check_attn_sync(m);
}

int qmh_model_time_prefill(qmh_model *m, const int32_t *tokens, int32_t n, int32_t pos0, int logits, double *ms) {
    if (!m || !tokens || n < 1 || pos0 < 0 || (int64_t)pos0 + n > m->cfg.max_seq || logits < 0 || logits > 2)
        return fail("time_prefill: bad arguments");
    for (int32_t i = 0; i < n; i++)
        if (tokens[i] < 0 || tokens[i] >= m->cfg.vocab_size) return fail("time_prefill: token %d out of range", tokens[i]);
    hipEvent_t e0, e1;
    HIPCHK(hipEventCreate(&e0));
    HIPCHK(hipEventCreate(&e1));
    hipError_t e = hipEventRecord(e0, g_stream);
    int rc = 0;
    if (e == hipSuccess) {
        if (m->pf_ok) {
            rc = pf_batched(m, tokens, n, pos0, logits, NULL);
        } else { /* the sequential path computes every position's logits anyway */
            for (int32_t i = 0; i < n && e == hipSuccess; i++) {
                int32_t *slot = m->h_tokpos + 4 * (size_t)i;
                slot[0] = tokens[i];
                slot[1] = pos0 + i;
                e = hipMemcpyAsync(m->d_tokpos, slot, sizeof(int32_t) * 2, hipMemcpyHostToDevice, g_stream);
                if (e == hipSuccess) e = run_step(m, 0, pos0 + i);
            }
        }
    }
    if (e == hipSuccess && rc == 0) e = hipEventRecord(e1, g_stream);
    if (e == hipSuccess && rc == 0) e = hipEventSynchronize(e1);
    float t = 0.0f;
    if (e == hipSuccess && rc == 0) e = hipEventElapsedTime(&t, e0, e1);
    hipEventDestroy(e0);
    hipEventDestroy(e1);
    if (rc) return -1;
    if (e != hipSuccess) return fail("time_prefill: %s", hipGetErrorString(e));
    if (ms) *ms = (double)t;
    return check_attn_sync(m);
}

int qmh_model_time_forward(qmh_model *m, int32_t token, int32_t pos, int32_t n_steps, int32_t *out, double *ms) {
    if (!m || n_steps < 1 || token < 0 || token >= m->cfg.vocab_size || pos < 0 ||
        (int64_t)pos + n_steps > m->cfg.max_seq)
        return fail("time_forward: bad token/range");
    const int V = m->cfg.vocab_size;
    struct timespec t0, t1;
    clock_gettime(CLOCK_MONOTONIC, &t0);
    int32_t tok = token;
    for (int32_t k = 0; k < n_steps; k++) {
        const float *lg = qmh_model_forward(m, tok, pos + k);
        if (!lg) return -1;
        int best = 0; /* qm_argmax (src/sampler.c:27-32) on the host, as bench/bench.c:147 does */
        for (int i = 1; i < V; i++)
            if (lg[i] > lg[best]) best = i;
        tok = best;
        if (out) out[k] = tok;
    }
    clock_gettime(CLOCK_MONOTONIC, &t1);
    if (ms) *ms = (double)(t1.tv_sec - t0.tv_sec) * 1e3 + (double)(t1.tv_nsec - t0.tv_nsec) * 1e-6;
    return 0;
}

/* ------------------------------------------------------------------ batched decode */

/* B independent sequences over one model's weights: each has its own KV cache (layout per layer
 * [seq][kvd][max_seq] for K, [seq][max_seq][kvd] for V); a step runs the B tokens through the
 * prefill kernels as one batch, with attention per sequence. */
struct qmh_batch {
    qmh_model *m;
    int32_t n;
    float *d_kt, *d_v;
    int32_t *d_tok, *d_pos, *d_record;
    int32_t *h_io; /* pinned [2n]: tokens, positions */
    int record_cap;
};

void qmh_batch_free(qmh_batch *b) {
    if (!b) return;
    void *bufs[] = {b->d_kt, b->d_v, b->d_tok, b->d_pos, b->d_record};
    for (size_t i = 0; i < sizeof bufs / sizeof bufs[0]; i++)
        if (bufs[i]) hipFree(bufs[i]);
    if (b->h_io) hipHostFree(b->h_io);
    free(b);
}

qmh_batch *qmh_batch_create(qmh_model *m, int32_t n_seq) {
    if (!m) {
        fail("batch: NULL model");
        return NULL;
    }
    if (!m->pf_ok) {
        fail("batch: needs quantized weights and head_dim <= 128, a multiple of 4 (the batched matmul path)");
        return NULL;
    }
    if (n_seq < 1 || n_seq > m->pf_cap) {
        fail("batch: n_seq %d outside [1, %d]", (int)n_seq, m->pf_cap);
        return NULL;
    }
    qmh_batch *b = calloc(1, sizeof *b);
    if (!b) {
        fail("batch: out of host memory");
        return NULL;
    }
    const qmh_config *c = &m->cfg;
    const size_t kv = (size_t)c->n_layers * n_seq * m->kvd * c->max_seq;
    b->m = m;
    b->n = n_seq;
    b->record_cap = c->max_seq;
    hipError_t e = hipMalloc((void **)&b->d_kt, kv * sizeof(float));
    if (e == hipSuccess) e = hipMalloc((void **)&b->d_v, kv * sizeof(float));
    if (e == hipSuccess) e = hipMalloc((void **)&b->d_tok, sizeof(int32_t) * (size_t)n_seq);
    if (e == hipSuccess) e = hipMalloc((void **)&b->d_pos, sizeof(int32_t) * (size_t)n_seq);
    if (e == hipSuccess) e = hipMalloc((void **)&b->d_record, sizeof(int32_t) * (size_t)n_seq * c->max_seq);
    if (e == hipSuccess) e = hipHostMalloc((void **)&b->h_io, sizeof(int32_t) * 2 * (size_t)n_seq, hipHostMallocDefault);
    if (e == hipSuccess) e = hipMemsetAsync(b->d_kt, 0, kv * sizeof(float), g_stream);
    if (e == hipSuccess) e = hipMemsetAsync(b->d_v, 0, kv * sizeof(float), g_stream);
    if (e == hipSuccess) e = hipStreamSynchronize(g_stream);
    if (e != hipSuccess) {
        fail("batch: %s", hipGetErrorString(e));
        qmh_batch_free(b);
        return NULL;
    }
    return b;
}

static int batch_check(const qmh_batch *b, const int32_t *tokens, const int32_t *pos, int32_t steps, int *max_pos) {
    const qmh_config *c = &b->m->cfg;
    *max_pos = 0;
    for (int32_t i = 0; i < b->n; i++) {
        if (tokens[i] < 0 || tokens[i] >= c->vocab_size) return fail("batch: sequence %d token %d out of range", i, tokens[i]);
        if (pos[i] < 0 || (int64_t)pos[i] + steps > c->max_seq)
            return fail("batch: sequence %d position %d (+%d steps) outside [0, %d)", i, pos[i], steps, c->max_seq);
        if (pos[i] > *max_pos) *max_pos = pos[i];
    }
    return 0;
}

/* one step: embed, the layers, and the logits of all sequences into d_pf_logits */
static int batch_step(qmh_batch *b, int max_pos, hipStream_t s) {
    qmh_model *m = b->m;
    const qmh_config *c = &m->cfg;
    const int D = c->dim, V = c->vocab_size, B = b->n;
    pf_seqs bt = {b->d_pos, max_pos, b->d_kt, b->d_v, (long long)m->kvd * c->max_seq};
    LCHK(qmh_launch_pf_embed(m->d_embd, m->emb_dtype, D, V, b->d_tok, B, m->d_pf_x, s));
    for (int l = 0; l < c->n_layers; l++)
        if (pf_layer(m, l, B, 0, &bt, s)) return -1;
    qmh_pf_args a;
    pf_args_for(m, &m->output, B, &a);
    a.xf = m->d_pf_x;
    a.ldxf = D;
    a.nxf = D;
    a.norm_w = m->d_norms + (size_t)(2 * c->n_layers) * D;
    a.eps = c->norm_eps;
    a.rows_alloc = m->output.ntiles * m->output.tile_r;
    a.epi = QMH_PF_STORE;
    a.out0 = m->d_pf_logits;
    a.ld0 = V;
    LCHK(qmh_launch_pf_gemm(&a, s));
    return 0;
}

int qmh_batch_forward(qmh_batch *b, const int32_t *tokens, const int32_t *pos, float *logits) {
    if (!b || !tokens || !pos) return fail("batch_forward: NULL argument");
    int max_pos;
    if (batch_check(b, tokens, pos, 1, &max_pos)) return -1;
    const int B = b->n, V = b->m->cfg.vocab_size;
    memcpy(b->h_io, tokens, sizeof(int32_t) * (size_t)B);
    memcpy(b->h_io + B, pos, sizeof(int32_t) * (size_t)B);
    HIPCHK(hipMemcpyAsync(b->d_tok, b->h_io, sizeof(int32_t) * (size_t)B, hipMemcpyHostToDevice, g_stream));
    HIPCHK(hipMemcpyAsync(b->d_pos, b->h_io + B, sizeof(int32_t) * (size_t)B, hipMemcpyHostToDevice, g_stream));
    if (batch_step(b, max_pos, g_stream)) return -1;
    if (logits)
        HIPCHK(hipMemcpyAsync(logits, b->m->d_pf_logits, sizeof(float) * (size_t)B * V, hipMemcpyDeviceToHost,
                              g_stream));
    HIPCHK(hipStreamSynchronize(g_stream));
    return 0;
}

int qmh_batch_greedy(qmh_batch *b, const int32_t *tokens, const int32_t *pos, int32_t n_steps, int32_t *out,
                     double *ms) {
    if (!b || !tokens || !pos || n_steps < 0) return fail("batch_greedy: bad argument");
    int max_pos;
    if (batch_check(b, tokens, pos, n_steps, &max_pos)) return -1;
    const int B = b->n, V = b->m->cfg.vocab_size;
    memcpy(b->h_io, tokens, sizeof(int32_t) * (size_t)B);
    memcpy(b->h_io + B, pos, sizeof(int32_t) * (size_t)B);
    HIPCHK(hipMemcpyAsync(b->d_tok, b->h_io, sizeof(int32_t) * (size_t)B, hipMemcpyHostToDevice, g_stream));
    HIPCHK(hipMemcpyAsync(b->d_pos, b->h_io + B, sizeof(int32_t) * (size_t)B, hipMemcpyHostToDevice, g_stream));
    hipEvent_t e0 = NULL, e1 = NULL;
    if (ms) {
        HIPCHK(hipEventCreate(&e0));
        HIPCHK(hipEventCreate(&e1));
        HIPCHK(hipEventRecord(e0, g_stream));
    }
    int rc = 0;
    for (int32_t k = 0; k < n_steps && !rc; k++) {
        rc = batch_step(b, max_pos + k, g_stream);
        if (!rc) rc = qmh_launch_bt_argmax(b->m->d_pf_logits, B, V, b->d_tok, b->d_pos, b->d_record, k, g_stream)
                          ? fail("batch_greedy: argmax launch failed")
                          : 0;
    }
    if (!rc && ms) {
        HIPCHK(hipEventRecord(e1, g_stream));
        HIPCHK(hipEventSynchronize(e1));
        float f = 0.0f;
        HIPCHK(hipEventElapsedTime(&f, e0, e1));
        *ms = f;
    }
    if (e0) hipEventDestroy(e0);
    if (e1) hipEventDestroy(e1);
    if (rc) return -1;
    if (n_steps > 0 && out)
        HIPCHK(hipMemcpyAsync(out, b->d_record, sizeof(int32_t) * (size_t)n_steps * B, hipMemcpyDeviceToHost,
                              g_stream));
    HIPCHK(hipStreamSynchronize(g_stream));
    return 0;
}

/* ------------------------------------------------------------------ sampler */

/* qm_sampler (src/sampler.h:8-16) with its two arena arrays replaced by device scratch: the
 * exponentials / probabilities and the radix-sort key and index buffers. The rng state lives on
 * the device, so sampling never returns to the host. */
struct qmh_sampler {
    int32_t n_vocab;
    float temperature, top_p;
    int top_k;
    uint64_t *d_rng;
    double *d_diag;
    int32_t *d_out;
    float *d_p;
    uint32_t *d_key[2];
    int32_t *d_idx[2];
    void *d_ws; /* control block and chunk arrays of the multi-workgroup path */
    int force_serial; /* QMH_SAMPLER_SERIAL set at creation: every exact sum by the serial fallback */
};

/* the reference's greedy shortcut (src/sampler.c:52): no draw, the rng is left alone */
static int sampler_greedy(const qmh_sampler *s) { return s->temperature == 0.0f || s->top_k == 1; }

void qmh_sampler_free(qmh_sampler *s) {
    if (!s) return;
    void *bufs[] = {s->d_rng,    s->d_diag,   s->d_out,    s->d_p,   s->d_key[0],
                    s->d_key[1], s->d_idx[0], s->d_idx[1], s->d_ws};
    for (size_t i = 0; i < sizeof bufs / sizeof bufs[0]; i++)
        if (bufs[i]) hipFree(bufs[i]);
    free(s);
}

qmh_sampler *qmh_sampler_create(int32_t n_vocab, float temperature, int top_k, float top_p, uint64_t seed) {
    if (ensure()) return NULL;
    if (n_vocab < 1 || n_vocab > (1 << 24)) {
        fail("sampler: n_vocab %d outside [1, 2^24]", (int)n_vocab);
        return NULL;
    }
    qmh_sampler *s = calloc(1, sizeof *s);
    if (!s) {
        fail("sampler: out of host memory");
        return NULL;
    }
    /* parameter normalisation of qm_sampler_init (src/sampler.c:8-12) */
    s->n_vocab = n_vocab;
    s->temperature = temperature < 0 ? 0 : temperature;
    s->top_k = top_k < 0 ? 0 : top_k;
    s->top_p = (top_p <= 0 || top_p > 1) ? 1.0f : top_p;
    uint64_t rng = seed ? seed : 0x9e3779b97f4a7c15ULL;
    s->force_serial = getenv("QMH_SAMPLER_SERIAL") != NULL;
    const size_t n = (size_t)n_vocab;
    hipError_t e = hipMalloc((void **)&s->d_rng, sizeof(uint64_t));
    if (e == hipSuccess) e = hipMalloc((void **)&s->d_diag, 8 * sizeof(double));
    if (e == hipSuccess) e = hipMalloc((void **)&s->d_out, sizeof(int32_t));
    if (e == hipSuccess) e = hipMalloc((void **)&s->d_p, n * sizeof(float));
    for (int k = 0; k < 2 && e == hipSuccess; k++) {
        e = hipMalloc((void **)&s->d_key[k], n * sizeof(uint32_t));
        if (e == hipSuccess) e = hipMalloc((void **)&s->d_idx[k], n * sizeof(int32_t));
    }
    const size_t wsb = qmh_sample_ws_bytes(n_vocab);
    if (e == hipSuccess && wsb) e = hipMalloc(&s->d_ws, wsb);
    if (e == hipSuccess && wsb) e = hipMemsetAsync(s->d_ws, 0, wsb, g_stream);
    if (e == hipSuccess) e = hipMemcpyAsync(s->d_rng, &rng, sizeof rng, hipMemcpyHostToDevice, g_stream);
    if (e == hipSuccess) e = hipStreamSynchronize(g_stream);
    if (e != hipSuccess) {
        fail("sampler: %s", hipGetErrorString(e));
        qmh_sampler_free(s);
        return NULL;
    }
    return s;
}

static qmh_sample_args sample_args(const qmh_sampler *s, const float *logits) {
    qmh_sample_args a;
    memset(&a, 0, sizeof a);
    a.logits = logits;
    a.n = s->n_vocab;
    a.temperature = s->temperature;
    a.top_k = s->top_k;
    a.top_p = s->top_p;
    a.rng = s->d_rng;
    a.p = s->d_p;
    a.key0 = s->d_key[0];
    a.key1 = s->d_key[1];
    a.idx0 = s->d_idx[0];
    a.idx1 = s->d_idx[1];
    a.diag = s->d_diag;
    a.ws = s->d_ws;
    a.force_serial = s->force_serial;
    return a;
}

int qmh_sample(qmh_sampler *s, const float *logits, int32_t *out, void *stream) {
    if (ensure()) return -1;
    if (!s || !logits || !out) return fail("sample: NULL argument");
    if (sampler_greedy(s)) {
        LCHK(qmh_launch_argmax(logits, s->n_vocab, out, NULL, NULL, 0, S(stream)));
        return 0;
    }
    qmh_sample_args a = sample_args(s, logits);
    a.out = out;
    LCHK(qmh_launch_sample(&a, S(stream)));
    return 0;
}

int qmh_sample_noalloc(const float *logits, int32_t n_vocab, float temperature, int top_k, float top_p,
                       uint64_t *rng, int32_t *out, void *stream) {
    /* no implicit qmh_init here: it allocates (the library stream, a rope table) */
    if (!g_ready) return fail("sample_noalloc: call qmh_init first");
    if (!logits || !rng || !out) return fail("sample_noalloc: NULL argument");
    if (n_vocab < 1 || n_vocab > QMH_SAMPLE_NOALLOC_MAX_VOCAB)
        return fail("sample_noalloc: n_vocab %d outside [1, %d] (the size of the static scratch)", (int)n_vocab,
                    QMH_SAMPLE_NOALLOC_MAX_VOCAB);
    /* parameter normalisation of qm_sampler_init (src/sampler.c:8-12) */
    qmh_sampler s;
    memset(&s, 0, sizeof s);
    s.n_vocab = n_vocab;
    s.temperature = temperature < 0 ? 0 : temperature;
    s.top_k = top_k < 0 ? 0 : top_k;
    s.top_p = (top_p <= 0 || top_p > 1) ? 1.0f : top_p;
    if (sampler_greedy(&s)) {
        LCHK(qmh_launch_argmax(logits, n_vocab, out, NULL, NULL, 0, S(stream)));
        return 0;
    }
    void *base = NULL;
    LCHK(qmh_sample_scratch(&base));
    qmh_sample_args a = sample_args(&s, logits);
    a.rng = rng;
    a.out = out;
    a.diag = NULL;
    LCHK(qmh_launch_sample_scratch(&a, base, S(stream)));
    return 0;
}

int32_t qmh_sample_sync(qmh_sampler *s, const float *logits) {
    if (!s) return fail("sample: NULL sampler");
    if (qmh_sample(s, logits, s->d_out, NULL)) return -1;
    int32_t tok = -1;
    HIPCHK(hipMemcpyAsync(&tok, s->d_out, sizeof tok, hipMemcpyDeviceToHost, g_stream));
    HIPCHK(hipStreamSynchronize(g_stream));
    return tok;
}

int qmh_sampler_rng(const qmh_sampler *s, uint64_t *state) {
    if (!s || !state) return fail("sampler_rng: NULL argument");
    HIPCHK(hipMemcpyAsync(state, s->d_rng, sizeof *state, hipMemcpyDeviceToHost, g_stream));
    HIPCHK(hipStreamSynchronize(g_stream));
    return 0;
}

int qmh_sampler_diag(const qmh_sampler *s, double diag[8], float *probs) {
    if (!s || !diag) return fail("sampler_diag: NULL argument");
    HIPCHK(hipMemcpyAsync(diag, s->d_diag, 8 * sizeof(double), hipMemcpyDeviceToHost, g_stream));
    if (probs)
        HIPCHK(hipMemcpyAsync(probs, s->d_p, sizeof(float) * (size_t)s->n_vocab, hipMemcpyDeviceToHost, g_stream));
    HIPCHK(hipStreamSynchronize(g_stream));
    return 0;
}

int qmh_model_sample(qmh_model *m, qmh_sampler *s, int32_t token, int32_t pos, int32_t n_steps, int32_t *out) {
    if (!m || !s) return fail("model_sample: NULL argument");
    if (s->n_vocab != m->cfg.vocab_size)
        return fail("model_sample: sampler vocab %d != model vocab %d", (int)s->n_vocab, (int)m->cfg.vocab_size);
    if (sampler_greedy(s)) return qmh_model_greedy(m, token, pos, n_steps, out);
    if (n_steps < 0 || token < 0 || token >= m->cfg.vocab_size || pos < 0 || (int64_t)pos + n_steps > m->cfg.max_seq)
        return fail("model_sample: bad token/range");
    int32_t *slot = m->h_tokpos;
    slot[0] = token, slot[1] = pos, slot[2] = 0, slot[3] = 0;
    HIPCHK(hipMemcpyAsync(m->d_tokpos, slot, sizeof(int32_t) * 4, hipMemcpyHostToDevice, g_stream));
    qmh_sample_args a = sample_args(s, m->d_logits);
    a.tokpos = m->d_tokpos;
    a.record = m->d_record;
    a.record_cap = m->cfg.max_seq;
    for (int32_t k = 0; k < n_steps; k++) {
        HIPCHK(run_step(m, 0, pos + k));
        LCHK(qmh_launch_sample(&a, g_stream));
    }
    if (n_steps > 0 && out)
        HIPCHK(hipMemcpyAsync(out, m->d_record, sizeof(int32_t) * (size_t)n_steps, hipMemcpyDeviceToHost, g_stream));
    HIPCHK(hipStreamSynchronize(g_stream));
    return check_attn_sync(m);
}

/* ------------------------------------------------------------------ generator */

int qmh_gen_qlm(const char *path, const qmh_config *cfg, int wtype, uint64_t seed, int n_threads) {
    char err[256];
    if (!path || !cfg) return fail("gen: NULL argument");
    if (qmh_gen_qlm_impl(path, cfg, wtype, seed, n_threads, err, sizeof err)) return fail("%s", err);
    return 0;
}
