/* qmhip.h -- C-ABI of the MI355X (gfx950) HIP token loop for quillm.
 *
 * Plain C: pointers, sizes and int return codes; no C++ or torch types. Every entry point
 * names the reference interface it stands in for (file:line in the reference tree).
 *
 * Conventions (mirroring the reference's, see its src/model.h:32-36 and src/ops.h:23-34):
 *   - op-level functions take DEVICE pointers and a stream (NULL = the library's stream) and
 *     return 0, or -1 with a message in qmh_last_error(). They are asynchronous on the stream.
 *   - model-level functions take host arguments; forward returns model-owned (pinned host)
 *     logits, valid until the next call, or NULL on a bad token/pos, like the reference.
 *   - results are bitwise identical to the reference's scalar ISA path
 *     (src/kernels_scalar.c) and bitwise reproducible run to run.
 *   - nothing here allocates on the host heap per token; device memory is allocated at
 *     model creation only.
 */
#ifndef QMHIP_H
#define QMHIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* tensor dtypes, same codes as the reference's qm_dtype (src/qm_base.h:11-15) */
enum { QMH_F32 = 0, QMH_Q8_0 = 2, QMH_Q4_0 = 3 };

/* ------------------------------------------------------------------ runtime */

/* 1 if a gfx950 device is visible. Stands in for qm_cpu_supports(QM_ISA_HIP) next to the
 * ISA probe of src/cpu.c:39-49. */
int qmh_available(void);
/* Select a device and create the library stream. 0 or -1. Stands in for qm_kernels_select
 * (src/kernels_scalar.c:71-76) for the "hip" ISA. */
int qmh_init(int device);
/* Thread-local message for the last -1/NULL return. */
const char *qmh_last_error(void);
/* The library's HIP stream (a hipStream_t) -- lets callers order their own work after ours. */
void *qmh_stream(void);

/* device memory plumbing for callers that hold no HIP runtime of their own */
void *qmh_dev_alloc(size_t bytes);
int qmh_dev_free(void *p);
int qmh_memcpy_h2d(void *dst, const void *src, size_t bytes);
int qmh_memcpy_d2h(void *dst, const void *src, size_t bytes);
int qmh_memset(void *dst, int value, size_t bytes);
int qmh_sync(void);

/* ------------------------------------------------------------------ op level (device pointers) */

/* fp16 <-> fp32, elementwise over n values. qm_fp16_to_fp32 / qm_fp32_to_fp16 (src/fp16.c:6-56) */
int qmh_fp16_to_fp32(const uint16_t *h, float *f, int64_t n, void *stream);
int qmh_fp32_to_fp16(const float *f, uint16_t *h, int64_t n, void *stream);

/* rows x n floats -> rows rows of Q8_0 / Q4_0 blocks in the reference byte layout (34 / 18 B
 * per 32 values, zero padded). qm_quantize_row_q8 / qm_quantize_row_q4 (src/quant.c:55-85). */
int qmh_quantize_rows_q8(const float *x, void *y, int64_t rows, int64_t n, void *stream);
int qmh_quantize_rows_q4(const float *x, void *y, int64_t rows, int64_t n, void *stream);
/* one row of any dtype -> n floats. qm_row_to_f32 (src/quant.c:96-101) */
int qmh_row_to_f32(int dtype, const void *row, float *y, int64_t n, void *stream);

/* A weight matrix resident on the device, repacked from the reference's row layout
 * (qm_tensor rows of qm_row_bytes, src/ops.h:8-22) into the tile layout the matvec reads. */
typedef struct qmh_weight qmh_weight;
/* host_rows: rows x cols in the .qlm / qm_tensor layout. NULL on error. */
qmh_weight *qmh_weight_upload(int dtype, int64_t rows, int64_t cols, const void *host_rows);
void qmh_weight_free(qmh_weight *w);

/* y[rows] = W x. For quantized W, x is quantized to Q8_0 first and, if xq is not NULL, the
 * quantized blocks are also written there (reference layout). qm_matvec (src/ops.c:57-61)
 * with the per-row dot_f32 / dot_q8 / dot_q4 of src/kernels_scalar.c:6-34. */
int qmh_matvec(const qmh_weight *W, const float *x, float *y, void *xq, void *stream);
/* y = W * rmsnorm(x, norm_w, eps) in one launch: the reference's qm_rmsnorm followed by
 * qm_matvec on its output (src/model.c:165-168,182-183), the fused kernel the model runs.
 * xq as for qmh_matvec (the quantized normalised activation). */
int qmh_rmsnorm_matvec(const qmh_weight *W, const float *x, const float *norm_w, float eps, float *y, void *xq,
                       void *stream);

/* C[M,N] = A[M,K] B[N,K]^T, all row-major contiguous f32. qm_matmul_nt (src/ops.c:81-90) ->
 * gemm_nt (src/gemm_driver.h:7-28), scalar-ISA rounding order (K panels of 256). */
int qmh_matmul_nt(const float *A, const float *B, float *C, int64_t M, int64_t N, int64_t K, void *stream);

/* elementwise ops of src/ops.c:93-133 (in-place where the reference is in place) */
int qmh_rmsnorm(float *out, const float *x, const float *w, int64_t n, float eps, void *stream);
int qmh_softmax(float *x, int64_t n, void *stream);
int qmh_rope(float *v, int64_t n_heads, int64_t head_dim, int64_t pos, float theta, void *stream);
int qmh_swiglu(float *gate, const float *up, int64_t n, void *stream);
/* *out = first index of the maximum. qm_argmax (src/sampler.c:27-32) */
int qmh_argmax(const float *x, int32_t n, int32_t *out, void *stream);

/* ------------------------------------------------------------------ model level (host arguments) */

/* qm_config (src/model.h:8-11) */
typedef struct {
    int32_t dim, hidden_dim, n_layers, n_heads, n_kv_heads, vocab_size, max_seq;
    float rope_theta, norm_eps;
} qmh_config;

/* A host tensor as the reference's qm_tensor describes it (src/ops.h:9-15): dtype, shape
 * (ne[0] outermost) and a pointer to rows of qm_row_bytes. */
typedef struct {
    int32_t dtype;
    int32_t ndim;
    int64_t ne[4];
    const void *data;
} qmh_tensor_view;

typedef struct qmh_model qmh_model;

/* Build the device model from host tensors the caller already holds (the reference's
 * qm_model after qm_model_load, src/model.c:35-117). layers[9*l + k] is layer l's
 * {attn_norm, wq, wk, wv, wo, ffn_norm, w1, w2, w3}[k] (src/model.h:13-15). Shapes are
 * validated as src/model.c:20-32,48-77 do. cfg->max_seq sizes the KV cache. NULL on error. */
qmh_model *qmh_model_create(const qmh_config *cfg, const qmh_tensor_view *tok_embd, const qmh_tensor_view *norm,
                            const qmh_tensor_view *output, const qmh_tensor_view *layers);
/* Open a .qlm file (format of src/qlm_file.h:1-9) and create the device model from it.
 * max_seq <= 0 keeps the file's context, else caps it (src/model.c:53). NULL on error. */
qmh_model *qmh_model_load(const char *path, int32_t max_seq);
void qmh_model_free(qmh_model *m);
const qmh_config *qmh_model_config(const qmh_model *m);
/* The configuration a .qlm file gives the model, read and validated as qm_model_load does
 * before it touches tensors (src/model.c:35-53: the seven u32 keys, rope_theta / norm_eps with
 * their defaults, the head checks, the max_seq cap; the first entry of a duplicated key wins, as
 * qlm_find_kv's does, src/qlm_file.c:181-185). Needs no device. 0, or -1 with a message. */
int qmh_qlm_config(const char *path, int32_t max_seq, qmh_config *out);

/* One token at position pos; returns model-owned logits[vocab] in pinned host memory, or
 * NULL for token outside [0, vocab) or pos outside [0, max_seq). qm_model_forward
 * (src/model.c:158-191). */
float *qmh_model_forward(qmh_model *m, int32_t token, int32_t pos);

/* n tokens at positions pos0..pos0+n-1, enqueued as one batch with no host round trip between
 * positions. KV cache contents and logits are bitwise those of n sequential qmh_model_forward
 * calls (the reference's prompt loop, src/main.c:127-130). logits: NULL, or host memory for
 * n*vocab floats. 0 or -1. */
int qmh_model_prefill(qmh_model *m, const int32_t *tokens, int32_t n, int32_t pos0, float *logits);

/* Greedy decode on the device: n_steps forwards starting with token at pos, each next token
 * the first argmax of the previous logits (reference bench/bench.c:143-149). out[k], k < n_steps,
 * receives the argmax of the logits of the forward at position pos+k (the token fed at pos+k+1).
 * No host round trip between steps. */
int qmh_model_greedy(qmh_model *m, int32_t token, int32_t pos, int32_t n_steps, int32_t *out);

/* ------------------------------------------------------------------ batched decode (bs > 1) */

/* n_seq independent sequences decoded together over one model's weights (no reference counterpart:
 * the reference decodes one sequence, src/model.c:158-191). Each sequence has its own KV cache of
 * the model's max_seq positions, separate from the model's own. Per sequence, logits and KV contents
 * are bitwise those of the single-sequence qmh_model_forward at the same tokens and positions.
 * Needs quantized weights and head_dim <= 128, a multiple of 4; n_seq in [1, min(max_seq, 512)]. NULL on error. */
typedef struct qmh_batch qmh_batch;
qmh_batch *qmh_batch_create(qmh_model *m, int32_t n_seq);
void qmh_batch_free(qmh_batch *b);
/* One step: sequence i takes tokens[i] at position pos[i] (any mix of positions). logits: NULL, or
 * host memory for n_seq x vocab floats. Synchronous. 0 or -1. */
int qmh_batch_forward(qmh_batch *b, const int32_t *tokens, const int32_t *pos, float *logits);
/* n_steps greedy steps of every sequence on the device, from tokens[i] at pos[i]: out[k*n_seq + i]
 * is sequence i's argmax after step k (the token it takes at step k+1). ms (optional): device time
 * of the n_steps steps from HIP events. 0 or -1. */
int qmh_batch_greedy(qmh_batch *b, const int32_t *tokens, const int32_t *pos, int32_t n_steps, int32_t *out,
                     double *ms);

/* ------------------------------------------------------------------ sampler */

/* qm_sampler (src/sampler.h:8-16): temperature / top-k / top-p sampling with an xorshift64*
 * stream. Results are token for token and rng state for rng state those of the reference's
 * qm_sample on the same logits (its float and double roundings included). */
typedef struct qmh_sampler qmh_sampler;

/* qm_sampler_init (src/sampler.c:6-16): the same normalisation (temperature < 0 -> 0, top_k < 0
 * -> 0, top_p outside (0, 1] -> 1, seed 0 -> 0x9e3779b97f4a7c15); device scratch replaces the
 * arena arrays. n_vocab in [1, 2^24]. NULL on error. */
qmh_sampler *qmh_sampler_create(int32_t n_vocab, float temperature, int top_k, float top_p, uint64_t seed);
void qmh_sampler_free(qmh_sampler *s);
/* qm_sample (src/sampler.c:50-106) of device logits[n_vocab]: the token is written to device
 * memory *out, asynchronously on the stream. Greedy configurations (temperature 0 or top_k 1)
 * take the first argmax and leave the rng alone, as the reference does. */
int qmh_sample(qmh_sampler *s, const float *logits, int32_t *out, void *stream);
/* qmh_sample on the library stream, synchronously: the token, or -1 on error. */
int32_t qmh_sample_sync(qmh_sampler *s, const float *logits);
/* The rng state (qm_sampler.rng) after the library stream's work. */
int qmh_sampler_rng(const qmh_sampler *s, uint64_t *state);
/* Diagnostics of the last non-greedy draw (no reference counterpart): diag[0] the serial double
 * sum of the exponentials, [1] 0 when every chunk certificate held, else nonzero: the sums were
 * then recomputed by one serial pass (as they are for every draw of a sampler created while the
 * environment variable QMH_SAMPLER_SERIAL is set), so the token stays exact, [2] chunks replayed serially
 * for that sum, [3] candidates, [4] k, [5] nucleus size m, [6] chunks replayed for the nucleus
 * sum, [7] nucleus mass. probs (NULL or host [n_vocab]): the normalised probabilities. */
int qmh_sampler_diag(const qmh_sampler *s, double diag[8], float *probs);

/* qmh_sample without a sampler object, allocating nothing: no counterpart in the reference. It is
 * for callers that cannot allocate device memory (code under HIP graph capture, serving loops).
 * The same draw as qmh_sample with a sampler created by qmh_sampler_create from these parameters;
 * *rng (device memory) holds the xorshift64* state and is advanced in place,
 * *out (device) receives the token, asynchronously on the stream (NULL = the library's). Scratch:
 * one static device array of 3186944 bytes per GPU, held until the process ends, so n_vocab is at
 * most 131072 (-1 otherwise). Calls that overlap on one GPU race on that array. qmh_init must have
 * run. 0 or -1. */
int qmh_sample_noalloc(const float *logits, int32_t n_vocab, float temperature, int top_k, float top_p,
                       uint64_t *rng, int32_t *out, void *stream);

/* Sampled decode on the device: n_steps forwards starting with token at pos, each next token
 * qm_sample of the previous logits (the generation loop of src/main.c:131-141). out[k] receives
 * the token sampled from the logits at position pos+k. No host round trip between steps. EOS does
 * not stop the loop (the reference stops there: cut out[] at the first EOS for its output). */
int qmh_model_sample(qmh_model *m, qmh_sampler *s, int32_t token, int32_t pos, int32_t n_steps, int32_t *out);

/* ------------------------------------------------------------------ measurement
 * No reference counterpart (the reference times with a host clock, bench/bench.c:11-38).
 * Stages of one decode step: 0 = fused RMSNorm+QKV matvec (+RoPE, KV write), 1 = Wo matvec
 * (+residual), 2 = fused RMSNorm+W1|W3 matvec (+SwiGLU), 3 = W2 matvec (+residual), 4 = final
 * RMSNorm+output matvec, 5 = attention scores, 6 = softmax + attention-weighted V sum, 7 = the
 * whole attention in one launch (scores, softmax and V sum; what decode steps use for positions below
 * 640, and below 1024 for head_dim 64 and 128, when the model's head shape allows it; an error for
 * other models and positions). */

/* Average device time of `iters` back-to-back launches of one stage at position pos (token 0),
 * from HIP events on the library stream; launch i uses layer i % n_layers, so weight reads come
 * from HBM rather than a cache. bytes_per_launch: weight bytes one launch streams (0 for
 * attention). Overwrites the KV cache entries at pos. */
int qmh_model_time_stage(qmh_model *m, int which, int32_t pos, int iters, double *ms_per_launch,
                         double *bytes_per_launch);
/* The reference bench's kernel rows (bench/bench.c:63-123, which time qm_matvec and qm_matmul_nt with
 * a host clock) on the device: the average device time (HIP events on the library stream) of `iters`
 * back-to-back qmh_matvec calls, call i on W[i % nw] (weights of one dtype and shape: several
 * copies make the reads come from HBM rather than a cache), and of qmh_matmul_nt calls. 0 or -1. */
int qmh_time_matvec(const qmh_weight *const *W, int nw, const float *x, float *y, int iters, double *ms_per_call);
int qmh_time_matmul_nt(const float *A, const float *B, float *C, int64_t M, int64_t N, int64_t K, int iters,
                       double *ms_per_call);
/* qmh_model_greedy, with HIP events around the n_steps graph replays (*ms = their total). */
int qmh_model_time_greedy(qmh_model *m, int32_t token, int32_t pos, int32_t n_steps, int32_t *out, double *ms);
/* qmh_model_prefill of n tokens at pos0, with HIP events around it (*ms). logits: 0 none, 1 the last
 * position's, 2 every position's (the reference's prompt loop computes them all: src/main.c:127-130);
 * they stay in device memory. */
int qmh_model_time_prefill(qmh_model *m, const int32_t *tokens, int32_t n, int32_t pos0, int logits, double *ms);
/* The reference bench's decode loop (bench/bench.c:143-149) on this model: n_steps of
 * token = argmax(qmh_model_forward(token, pos + k)), the argmax on the host over the returned (copied)
 * logits; *ms from a host clock; out (optional) receives the tokens. */
int qmh_model_time_forward(qmh_model *m, int32_t token, int32_t pos, int32_t n_steps, int32_t *out, double *ms);

/* ------------------------------------------------------------------ synthetic models */

/* Write a random-init .qlm (format src/qlm_file.h:1-9, tensor order of the reference's
 * writer): every 2-D tensor ~ N(0, 0.02) from a counter-based generator keyed by (seed,
 * tensor, element) and stored as wtype; norm gains 1.0. Results do not depend on n_threads.
 * 0 or -1. No reference counterpart in C (the reference's generator is its Python tooling). */
int qmh_gen_qlm(const char *path, const qmh_config *cfg, int wtype, uint64_t seed, int n_threads);
/* The f32 values (before quantization) of elements [k0, k0+n) of tensor number tensor_index
 * (its position in the file's tensor table) of a model written by qmh_gen_qlm with `seed`;
 * lets a checker re-quantize them with another quantizer. */
void qmh_gen_values(uint64_t seed, int tensor_index, int64_t k0, int64_t n, float *out);

#ifdef __cplusplus
}
#endif
#endif
