/* CPU oracle for the quillm token loop -- TEST INFRASTRUCTURE ONLY.
 *
 * A plain C11 restatement of the reference's scalar CPU path (the arithmetic of
 * src/fp16.c, src/quant.c, src/kernels_scalar.c, src/gemm_driver.h, src/ops.c,
 * src/model.c, src/sampler.c), written independently and compiled with the same float
 * semantics as the reference (ISO C, no contraction, no FMA, no fast-math), so every
 * result is bit-identical to the reference's scalar ISA.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load this
 * library, and only as the checker. The product (quillm_amd/) never links it.
 *
 * Pinning (each function is checked by tests/test_oracle_*.py against something other
 * than its own formula):
 *   or_h2f/or_f2h        exhaustive 65,536 round trip, the reference's KATs
 *                        (tests/test_fp16.c:29-38), numpy float16 (IEEE RNE), and a strided
 *                        2^32 sweep against the compiled reference (oracle/_ref).
 *   or_quantize_*        byte-exact against the compiled reference on random rows, KATs of
 *                        tests/test_quant.c:61-75 and tests/test_python.py:32-36.
 *   or_dot_*             bit-exact against the compiled reference's scalar kernels, and
 *                        within accum_tol of a float64 brute force (tests/test_kernels.c:13).
 *   or_gemm_nt           bit-exact against the compiled reference's scalar gemm_nt, and
 *                        within accum_tol of float64 brute force.
 *   or_rmsnorm..swiglu   bit-exact against the compiled reference, plus the closed forms of
 *                        tests/test_kernels.c:104-138.
 *   or_argmax            KAT of tests/test_sampler.c:8-12.
 *   or_sample            token sequences and rng states identical to the compiled reference's
 *                        qm_sample on seeded logits (every parameter path, NaN/inf logits,
 *                        ties), the KATs of tests/test_sampler.c, and its distribution checks
 *                        against softmax(logits/T) in float64.
 *   or_model_forward     bit-exact logits against the compiled reference's qm_model_forward
 *                        (scalar ISA) on generated .qlm files; causality.
 */
#ifndef QM_ORACLE_H
#define QM_ORACLE_H

#include <stddef.h>
#include <stdint.h>

/* dtypes as stored in .qlm (reference src/qm_base.h:11-15) */
enum { OR_F32 = 0, OR_Q8_0 = 2, OR_Q4_0 = 3 };

float or_h2f(uint16_t h);
uint16_t or_f2h(float f);
/* whole-array helpers for fast exhaustive checks */
void or_f2h_array(const float *x, uint16_t *y, int64_t n);
void or_h2f_array(const uint16_t *x, float *y, int64_t n);

int64_t or_nblocks(int64_t n);
size_t or_row_bytes(int dtype, int64_t n);
void or_quantize_q8(const float *x, uint8_t *out, int64_t n); /* out: nblocks*34 bytes */
void or_quantize_q4(const float *x, uint8_t *out, int64_t n); /* out: nblocks*18 bytes */
void or_row_to_f32(int dtype, const void *row, float *y, int64_t n);
/* rows x n, each row quantized independently (rows of row_bytes each) */
void or_quantize_rows(int dtype, const float *x, uint8_t *out, int64_t rows, int64_t n);

float or_dot_f32(const float *a, const float *b, int64_t n);
float or_dot_q8(const uint8_t *w, const uint8_t *x, int64_t nb);
float or_dot_q4(const uint8_t *w, const uint8_t *x, int64_t nb);
void or_gemm_nt(const float *A, const float *B, float *C, int64_t M, int64_t N, int64_t K, int64_t lda,
                int64_t ldb, int64_t ldc);
/* y[rows] = W x, with x quantized into xq first when W is quantized (reference src/ops.c:57-61) */
void or_matvec(int dtype, const void *W, int64_t rows, int64_t cols, const float *x, float *y, uint8_t *xq);

void or_rmsnorm(float *out, const float *x, const float *w, int64_t n, float eps);
void or_softmax(float *x, int64_t n);
void or_rope(float *v, int64_t n_heads, int64_t head_dim, int64_t pos, float theta);
void or_swiglu(float *gate, const float *up, int64_t n);
int32_t or_argmax(const float *x, int32_t n);

/* ---- sampler (reference src/sampler.{h,c}) ---- */
typedef struct {
    float temperature;
    int top_k;
    float top_p;
    uint64_t rng;
    int32_t n_vocab;
} or_sampler;
void or_sampler_init(or_sampler *s, int32_t n_vocab, float temperature, int top_k, float top_p, uint64_t seed);
float or_rng_uniform(uint64_t *state);
/* q[n], order[n]: caller's work space (q ends as the normalised probabilities, order as the
 * sorted candidates); *sum_out (optional) gets the serial double sum of the exponentials. */
int32_t or_sample(or_sampler *s, const float *logits, float *q, int32_t *order, double *sum_out);

/* ---- model (reference src/model.{h,c}) ---- */
typedef struct or_model or_model;
/* max_seq <= 0 keeps the file's value. Returns NULL and fills err on failure. */
or_model *or_model_load(const char *path, int max_seq, char *err, size_t errlen);
void or_model_free(or_model *m);
/* NULL on bad token/pos, else model-owned logits[vocab] */
float *or_model_forward(or_model *m, int32_t token, int32_t pos);
/* dim, hidden, layers, heads, kv_heads, vocab, max_seq */
void or_model_dims(const or_model *m, int32_t out[7]);

#endif
