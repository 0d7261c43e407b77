/* Internal C interface between the C11 host code (quillm_amd/host) and the HIP kernels
 * (quillm_amd/csrc). Plain C types only; every launcher enqueues on `stream` (a
 * hipStream_t) and returns a hipError_t as int (0 = success). */
#ifndef QMH_LAUNCH_H
#define QMH_LAUNCH_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* rows per tile of the device weight layout */
#define QMH_TILE_R 16
/* slots of padding after a quantized weight's tiles: >= one matvec chunk (256 threads x 8 blocks) */
#define QMH_WEIGHT_PAD_SLOTS 4096

/* matvec epilogues */
enum {
    QMH_EPI_STORE = 0,  /* out0[row] = y */
    QMH_EPI_ADD = 1,    /* out0[row] = out0[row] + y  (residual, src/model.c:179,186) */
    QMH_EPI_QKV = 2,    /* rows [0,seg1): q with RoPE -> out0; [seg1,seg2): k with RoPE -> K cache
                           row pos (out1); [seg2,rows): v -> transposed V cache column pos (out2) */
    QMH_EPI_SWIGLU = 3, /* interleaved W1|W3 tiles: out0[row] = silu(y1)*y3 (src/ops.c:128-133) */
    QMH_EPI_SWIGLU_Q = 4, /* as SWIGLU with 64-row tiles (32 outputs = one Q8_0 block), and the block
                             quantized into the activation image xq_img for the next matvec */
};

/* Activation image: a vector quantized to Q8_0 in the layout the quantized matvec keeps in LDS,
 * [codes: nb*32 int8][d: nb fp32 (fp32(fp16(d)))][code sums: nb int32], padded to 16 bytes.
 * Codes are in element order, or split (even elements then odd) for a Q4_0 consumer. */
#define QMH_XQ_IMAGE_BYTES(nb) ((((size_t)(nb)) * 40 + 15) & ~(size_t)15)

typedef struct {
    /* weight: tiled codes/scales (quantized) or row-major floats (f32) */
    int dtype;
    const void *codes;
    const uint16_t *scales;
    int nb;      /* blocks per row (quantized) */
    int cols;    /* elements per row */
    int tile_r;  /* rows per tile: 8 or 16, or 32 / 64 for interleaved W1|W3 */
    int ntiles;
    int rows;    /* valid output rows (per half for the interleaved W1|W3) */
    /* activation: x[cols]; optional RMSNorm gain (norm_w != NULL) applied before quantization */
    const float *x;
    const float *norm_w;
    float eps;
    uint8_t *xq_out; /* optional: quantized activation in the reference Q8_0 layout */
    const void *xq_in; /* instead of x: the activation already quantized, as an image */
    void *xq_img;      /* SWIGLU_Q: the output image (xq_nb blocks), codes split when xq_split */
    int xq_nb, xq_split;
    /* epilogue */
    int epi;
    float *out0, *out1, *out2;
    int seg1, seg2;
    const float *rope; /* [max_seq][head_dim/2][2] (cos, sin) */
    const int32_t *pos_ptr;
    int head_dim, max_seq, kvd;
    int exact_norm; /* tests: the RMSNorm always takes the serial sum of squares */
} qmh_mv_args;

/* nslots: slots the codes/scales allocation holds; slots at or past it are never written */
int qmh_launch_repack(const uint8_t *src, int64_t src_rows, int nb, int dtype, uint8_t *codes, uint16_t *scales,
                      int tile_r, int64_t row_off, int interleave_half, int64_t nslots, void *stream);
/* quantized matvec (k_matvec): grid from qmh_matvec_grid (want: workgroups wanted, about one
 * per CU; returns -1 if one tile does not fit the workgroup's LDS) */
int qmh_matvec_grid(int ntiles, int nb, int tile_r, int dtype, int want);
int qmh_launch_matvec(const qmh_mv_args *a, int grid, void *stream);
/* longest row the quantized matvec takes, with (norm = 1) or without the RMSNorm prologue */
int qmh_matvec_max_cols(int norm);
int qmh_matvec_max_image_cols(void);
/* f32 weights: plain rows, serial dot per row (src/kernels_scalar.c:6-10) */
int qmh_launch_matvec_f32(const qmh_mv_args *a, void *stream);

/* step_ctr (may be NULL): a decode-step counter the kernel adds one to (k_attn_fused's epochs) */
int qmh_launch_embed(const uint8_t *tok_embd, int dtype, int dim, int vocab, const int32_t *tok_ptr, float *x,
                     uint32_t *step_ctr, void *stream);
int qmh_launch_attn_scores(const float *q, const float *kcache, float *att, const int32_t *pos_ptr, int n_heads,
                           int n_kv_heads, int head_dim, int max_seq, float scale, void *stream);
/* the same scores for a kv head serving several query heads: K tile in LDS (head_dim 48, 64 or
 * 128, max_seq % 4 == 0); qmh_launch_attn_scores calls it */
int qmh_launch_attn_scores_tile(const float *q, const float *kcache, float *att, const int32_t *pos_ptr, int n_heads,
                                int n_kv_heads, int head_dim, int max_seq, float scale, void *stream);
int qmh_launch_attn_pv(const float *att, const float *vtcache, float *out, const int32_t *pos_ptr, int n_heads,
                       int n_kv_heads, int head_dim, int max_seq, void *stream);
/* a decode step's attention in one launch (k_attn_fused) for contexts of up to
 * qmh_attn_fused_max_n(instance) positions (instance 0: 640, 1: 1024): scores exchanged between a
 * head's workgroups as epoch-tagged words in attp [n_heads][max_seq] (zeroed at allocation); sync[0]
 * counts decode steps (qmh_launch_embed), sync[1] != 0 reports a bounded wait that ran out (or a
 * launch past the instance's context limit). Each workgroup owns cw output columns of a head (16
 * or 8; qmh_attn_fused_cw: the width for the shape on this device). qmh_attn_fused_supported: how
 * many instances take the shape at that width (0, 1 or 2) */
int qmh_attn_fused_max_n(int instance);
int qmh_attn_fused_cw(int n_heads, int head_dim);
int qmh_attn_fused_supported(int n_heads, int n_kv_heads, int head_dim, int max_seq, int cw);
int qmh_launch_attn_fused(const float *q, const float *kcache, const float *vcache, float *out, uint64_t *attp,
                          const int32_t *pos_ptr, uint32_t *sync, int n_heads, int n_kv_heads, int head_dim,
                          int max_seq, float scale, int layer, int n_layers, int instance, int cw, int stall,
                          void *stream);
/* the decode attention kernels over B sequences of a batched step (MHA, head_dim 128/64/48; else
 * hipErrorNotSupported): query Q[b][n_heads*hd], caches at Kt/V + b*kv_stride, position pos[b],
 * scores att[b][n_heads][max_seq], out[b][n_heads*hd] */
int qmh_launch_attn_batch(const float *Q, const float *Kt, const float *V, long long kv_stride, const int32_t *pos,
                          float *att, float *out, int B, int n_heads, int n_kv, int hd, int max_seq, float scale,
                          void *stream);
/* ---- batched prefill (qmh_prefill.hip) ---- */
enum { QMH_PF_STORE = 0, QMH_PF_ADD = 1, QMH_PF_QKV = 2, QMH_PF_SWIGLU = 3 };
/* token counts up to this run the skinny matmul (every weight streamed once for all tokens), larger
 * ones the tiled matmul */
#ifndef QMH_PF_SKINNY_P
#define QMH_PF_SKINNY_P 64
#endif
typedef struct {
    /* weight: tiled codes/scales as for the matvec; il: interleaved W1 | W3 tiles */
    int dtype;
    const uint8_t *codes;
    const uint16_t *scales;
    int nb, tile_r, il, rows, rows_alloc; /* rows: output rows; rows_alloc: rows with slots */
    /* activations: Q8_0 codes [nb][PP][32] and scales [nb][PP] of P tokens (PP % 128 == 0) */
    const int8_t *xc;
    const float *xd;
    int PP, P;
    /* or (xf != NULL) the f32 rows they come from: xf[p*ldxf + i], i < nxf, RMSNorm'd with gain norm_w
     * first when norm_w != NULL; the launcher quantizes them (inside the multi-token matvec, or into
     * xc/xd with k_pf_quant before the matmul) */
    const float *xf;
    int ldxf, nxf;
    const float *norm_w;
    float eps;
    /* epilogue: out0 row-major [P][ld0]; QKV: q -> out0, k -> out1 ([kvd][max_seq]), v -> out2 */
    int epi;
    /* SWIGLU through the tiled matmul (P > QMH_PF_SKINNY_P): with qxc set, the output is written only as the next
     * matmul's Q8_0 image, codes [nb][PP][32] (Q4_0 order when qperm8) and scales [nb][PP], instead of
     * out0 (the quantization the launcher would run on it, bit for bit) */
    int8_t *qxc;
    float *qxd;
    int qperm8;
    float *out0, *out1, *out2;
    int ld0, seg1, seg2;
    const float *rope;
    int pos0, head_dim, max_seq, kvd;
    /* QKV of independent sequences (batched decode): token p is at position pos_arr[p] and writes the
     * caches at out1/out2 + p*kv_stride; NULL / 0 for one prompt at positions pos0 + p */
    const int32_t *pos_arr;
    long long kv_stride;
    /* set by the matmul launcher: the multi-token matvec's blocks per LDS round (0: all at once) */
    int bmv_bq;
} qmh_pf_args;
int qmh_launch_pf_embed(const uint8_t *tok_embd, int dtype, int dim, int vocab, const int32_t *tokens, int P, float *X,
                        void *stream);
/* rows p < P of x (stride ldx, n values; RMSNorm'd with gain w when w != NULL) -> image codes/scales */
int qmh_launch_pf_quant(const float *x, int ldx, const float *w, float eps, int n, int P, int8_t *xc, float *xd,
                        int PP, int perm8, void *stream);
int qmh_launch_pf_gemm(const qmh_pf_args *a, void *stream);
/* causal attention of P tokens at positions pos0.. over the caches; att: scratch [n_heads][P][max_seq].
 * xc != NULL (head_dim 128 or 64 only): out is also written as its Q8_0 image (xc, xd, PP tokens per
 * block, perm8: the Q4_0 consumers' byte order), as qmh_launch_pf_quant would write it */
int qmh_launch_pf_attention(const float *Q, const float *Kt, const float *V, float *att, float *out, int P, int pos0,
                            int n_heads, int n_kv, int hd, int max_seq, float scale, int8_t *xc, float *xd, int PP,
                            int perm8, void *stream);

/* attention of B independent sequences, one query each (src/model.c:127-156 per sequence): sequence b
 * at position pos[b] (device), query Q[b][n_heads*hd], caches Kt + b*kv_stride ([kvd][max_seq]) and
 * V + b*kv_stride ([max_seq][kvd]); att: scratch [B][n_heads][max_seq]; out[b][n_heads*hd].
 * max_pos: the largest pos[b] (sizes the grid and the LDS). split == 0: up to 3 sequences of one query
 * head per kv head and head_dim 128/64/48 the decode kernels with a sequence dimension (through att),
 * else one fused kernel when max_pos < 16384 (att unused), else three launches through att;
 * split == 1: always three launches; split == 2: the fused kernel when max_pos < 16384 */
int qmh_launch_bt_attention(const float *Q, const float *Kt, const float *V, long long kv_stride, const int32_t *pos,
                            int max_pos, float *att, float *out, int B, int n_heads, int n_kv, int hd, int max_seq,
                            float scale, int split, void *stream);

/* per row b of logits[B][V]: tok[b] = first argmax, pos[b] += 1, record[step*B + b] = it (if record) */
int qmh_launch_bt_argmax(const float *logits, int B, int V, int32_t *tok, int32_t *pos, int32_t *record, int step,
                         void *stream);

/* argmax over x[n] -> *out_idx; if tokpos != NULL also tokpos[0] = idx, tokpos[1] += 1 and
 * record[step] = idx (when step < record_cap) where step = tokpos[2]++ (device greedy loop state) */
int qmh_launch_argmax(const float *x, int n, int32_t *out_idx, int32_t *tokpos, int32_t *record, int record_cap,
                      void *stream);
/* one qm_sample (src/sampler.c:50-106) of a non-greedy sampler: token -> *out (and the decode
 * loop's tokpos/record like qmh_launch_argmax); rng advanced in place. p: [n] scratch (ends as the
 * probabilities), key0/key1/idx0/idx1: [n] sort scratch; diag (optional, [8]): serial sum, status
 * (0 = every replayed chunk end matched), chunks replayed, candidates, k, m, chunks replayed in
 * the nucleus sum, nucleus mass. */
typedef struct {
    const float *logits;
    int n;
    float temperature;
    int top_k;
    float top_p;
    uint64_t *rng;
    float *p;
    uint32_t *key0, *key1;
    int32_t *idx0, *idx1;
    int32_t *out;
    int32_t *tokpos;
    int32_t *record;
    int record_cap;
    double *diag;
    void *ws; /* qmh_sample_ws_bytes(n) bytes, zeroed once at allocation (large vocabularies) */
    int force_serial; /* nonzero: both exact sums take the serial pass that a failed certificate takes */
} qmh_sample_args;
size_t qmh_sample_ws_bytes(int n);
int qmh_launch_sample(const qmh_sample_args *a, void *stream);
/* The sampler's static scratch (qmh_sample.hip): a file-scope device array of QMH_SAMPLE_NOALLOC_BYTES
 * holding p, key0/1, idx0/1 and the grid workspace for up to QMH_SAMPLE_NOALLOC_MAX_VOCAB entries.
 * qmh_sample_scratch: its device address on the current device (looked up once per device).
 * qmh_launch_sample_scratch: points a's buffers into it (base = that address) and launches the draw. */
#define QMH_SAMPLE_NOALLOC_MAX_VOCAB 131072
#define QMH_SAMPLE_NOALLOC_BYTES 3186944
int qmh_sample_scratch(void **ptr);
int qmh_launch_sample_scratch(qmh_sample_args *a, void *base, void *stream);

/* gate = silu(gate)*up over n (src/ops.c:128-133) */
int qmh_launch_swiglu(float *gate, const float *up, int64_t n, void *stream);

/* op-level kernels */
int qmh_launch_h2f(const uint16_t *h, float *f, int64_t n, void *stream);
int qmh_launch_f2h(const float *f, uint16_t *h, int64_t n, void *stream);
int qmh_launch_quantize_rows(const float *x, uint8_t *y, int64_t rows, int64_t n, int dtype, void *stream);
int qmh_launch_row_to_f32(const uint8_t *row, int dtype, float *y, int64_t n, void *stream);
int qmh_launch_rmsnorm(float *out, const float *x, const float *w, int64_t n, float eps, void *stream);
int qmh_launch_softmax(float *x, int64_t n, void *stream);
int qmh_launch_rope(float *v, int64_t n_heads, int64_t head_dim, const float *table, int64_t pos, void *stream);
int qmh_launch_gemm_nt(const float *A, const float *B, float *C, int64_t M, int64_t N, int64_t K, void *stream);

#ifdef __cplusplus
}
#endif
#endif
