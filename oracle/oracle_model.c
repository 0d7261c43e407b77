/* CPU oracle, model part -- TEST INFRASTRUCTURE ONLY (see oracle.h).
 * A minimal .qlm reader and the token forward of the reference (src/model.c:158-191). */
#include <fcntl.h>
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include "oracle.h"

typedef struct {
    char name[64];
    int dtype;
    int ndim;
    int64_t ne[4];
    const uint8_t *data;
} or_tensor;

typedef struct {
    const or_tensor *attn_norm, *wq, *wk, *wv, *wo, *ffn_norm, *w1, *w2, *w3;
} or_layer;

struct or_model {
    int32_t dim, hidden, n_layers, n_heads, n_kv_heads, vocab, max_seq;
    float theta, eps;
    uint8_t *map;
    size_t map_size;
    or_tensor *tensors;
    uint32_t n_tensors;
    const or_tensor *tok_embd, *norm, *output;
    or_layer *layers;
    float *x, *xb, *xb2, *q, *hb, *hb2, *att, *logits, *kc, *vc;
    uint8_t *xq;
};

/* ---- .qlm layout (reference src/qlm_file.h:1-9), little-endian ---- */
typedef struct {
    const uint8_t *p;
    size_t n, off;
    int bad;
} cur;

static const uint8_t *take(cur *c, size_t k) {
    if (c->bad || k > c->n - c->off) {
        c->bad = 1;
        return NULL;
    }
    const uint8_t *r = c->p + c->off;
    c->off += k;
    return r;
}
static uint32_t u32le(cur *c) {
    const uint8_t *b = take(c, 4);
    return b ? (uint32_t)b[0] | (uint32_t)b[1] << 8 | (uint32_t)b[2] << 16 | (uint32_t)b[3] << 24 : 0;
}
static uint64_t u64le(cur *c) {
    uint64_t lo = u32le(c);
    return lo | (uint64_t)u32le(c) << 32;
}
static int str(cur *c, char *dst, size_t cap) {
    uint32_t k = u32le(c);
    const uint8_t *s = (k && k < cap) ? take(c, k) : NULL;
    if (!s) return -1;
    memcpy(dst, s, k);
    dst[k] = 0;
    return 0;
}

static const or_tensor *find(const or_model *m, const char *name) {
    for (uint32_t i = 0; i < m->n_tensors; i++)
        if (!strcmp(m->tensors[i].name, name)) return &m->tensors[i];
    return NULL;
}

static int want(const or_model *m, const or_tensor **dst, const char *name, int64_t d0, int64_t d1) {
    const or_tensor *t = find(m, name);
    if (!t) return -1;
    if (d1 == 0 && !(t->ndim == 1 && t->ne[0] == d0 && t->dtype == OR_F32)) return -1;
    if (d1 != 0 && !(t->ndim == 2 && t->ne[0] == d0 && t->ne[1] == d1)) return -1;
    *dst = t;
    return 0;
}

or_model *or_model_load(const char *path, int max_seq, char *err, size_t errlen) {
    or_model *m = calloc(1, sizeof *m);
    int fd = open(path, O_RDONLY);
    struct stat st;
    if (!m || fd < 0 || fstat(fd, &st) != 0) {
        snprintf(err, errlen, "cannot open %s", path);
        if (fd >= 0) close(fd);
        free(m);
        return NULL;
    }
    m->map_size = (size_t)st.st_size;
    m->map = mmap(NULL, m->map_size, PROT_READ, MAP_PRIVATE, fd, 0);
    close(fd);
    if (m->map == MAP_FAILED) {
        snprintf(err, errlen, "mmap failed");
        free(m);
        return NULL;
    }
    cur c = {m->map, m->map_size, 0, 0};
    const uint8_t *mg = take(&c, 4);
    uint32_t ver = u32le(&c), n_kv = u32le(&c), n_t = u32le(&c);
    uint64_t data_off = u64le(&c);
    if (!mg || memcmp(mg, "QLMF", 4) || ver != 1 || c.bad || data_off > m->map_size || n_t > 4096) goto bad;
    m->theta = 10000.0f;
    m->eps = 1e-5f;
    for (uint32_t i = 0; i < n_kv; i++) {
        char key[64];
        if (str(&c, key, sizeof key)) goto bad;
        uint32_t ty = u32le(&c);
        uint32_t v = 0;
        if (ty == 0 || ty == 1) v = u32le(&c);
        else if (ty == 2) take(&c, u32le(&c));
        else if (ty == 3) {
            uint32_t cnt = u32le(&c);
            if (cnt > (m->map_size - c.off) / 4) goto bad;
            take(&c, (size_t)cnt * 4);
        } else goto bad;
        if (c.bad) goto bad;
        float fv;
        memcpy(&fv, &v, 4);
        struct { const char *k; int32_t *dst; } u32keys[] = {
            {"llama.dim", &m->dim}, {"llama.hidden_dim", &m->hidden}, {"llama.n_layers", &m->n_layers},
            {"llama.n_heads", &m->n_heads}, {"llama.n_kv_heads", &m->n_kv_heads}, {"llama.vocab_size", &m->vocab},
            {"llama.max_seq", &m->max_seq}};
        for (size_t k = 0; k < sizeof u32keys / sizeof u32keys[0]; k++)
            if (ty == 0 && !strcmp(key, u32keys[k].k)) *u32keys[k].dst = (int32_t)v;
        if (ty == 1 && !strcmp(key, "llama.rope_theta")) m->theta = fv;
        if (ty == 1 && !strcmp(key, "llama.norm_eps")) m->eps = fv;
    }
    m->tensors = calloc(n_t ? n_t : 1, sizeof(or_tensor));
    m->n_tensors = n_t;
    for (uint32_t i = 0; i < n_t; i++) {
        or_tensor *t = &m->tensors[i];
        if (str(&c, t->name, sizeof t->name)) goto bad;
        t->dtype = (int)u32le(&c);
        t->ndim = (int)u32le(&c);
        if (t->ndim < 1 || t->ndim > 4) goto bad;
        for (int d = 0; d < t->ndim; d++) t->ne[d] = (int64_t)u64le(&c);
        uint64_t off = u64le(&c);
        int64_t rows = 1;
        for (int d = 0; d + 1 < t->ndim; d++) rows *= t->ne[d];
        size_t bytes = (size_t)rows * or_row_bytes(t->dtype, t->ne[t->ndim - 1]);
        if (c.bad || data_off + off + bytes > m->map_size) goto bad;
        t->data = m->map + data_off + off;
    }
    if (!m->dim || !m->hidden || !m->n_layers || !m->n_heads || !m->n_kv_heads || !m->vocab || !m->max_seq ||
        m->dim % m->n_heads || m->n_heads % m->n_kv_heads || (m->dim / m->n_heads) % 2)
        goto bad;
    if (max_seq > 0 && max_seq < m->max_seq) m->max_seq = max_seq;
    int64_t D = m->dim, H = m->hidden, KV = (int64_t)m->dim / m->n_heads * m->n_kv_heads, V = m->vocab;
    m->layers = calloc((size_t)m->n_layers, sizeof(or_layer));
    if (want(m, &m->tok_embd, "tok_embd", V, D) || want(m, &m->norm, "norm", D, 0) || want(m, &m->output, "output", V, D))
        goto bad;
    for (int l = 0; l < m->n_layers; l++) {
        char nm[64];
        or_layer *L = &m->layers[l];
        struct { const or_tensor **dst; const char *sfx; int64_t d0, d1; } ws[] = {
            {&L->attn_norm, "attn_norm", D, 0}, {&L->wq, "wq", D, D},  {&L->wk, "wk", KV, D},
            {&L->wv, "wv", KV, D},              {&L->wo, "wo", D, D},  {&L->ffn_norm, "ffn_norm", D, 0},
            {&L->w1, "w1", H, D},               {&L->w2, "w2", D, H}, {&L->w3, "w3", H, D}};
        for (size_t k = 0; k < sizeof ws / sizeof ws[0]; k++) {
            snprintf(nm, sizeof nm, "layers.%d.%s", l, ws[k].sfx);
            if (want(m, ws[k].dst, nm, ws[k].d0, ws[k].d1)) goto bad;
        }
    }
    int64_t S = m->max_seq, maxdim = D > H ? D : H;
    m->x = calloc((size_t)D, 4);
    m->xb = calloc((size_t)D, 4);
    m->xb2 = calloc((size_t)D, 4);
    m->q = calloc((size_t)D, 4);
    m->hb = calloc((size_t)H, 4);
    m->hb2 = calloc((size_t)H, 4);
    m->att = calloc((size_t)S, 4);
    m->logits = calloc((size_t)V, 4);
    m->kc = calloc((size_t)m->n_layers * S * KV, 4);
    m->vc = calloc((size_t)m->n_layers * S * KV, 4);
    m->xq = calloc((size_t)or_nblocks(maxdim), 34);
    if (!m->kc || !m->vc || !m->xq) {
        snprintf(err, errlen, "out of memory");
        or_model_free(m);
        return NULL;
    }
    return m;
bad:
    snprintf(err, errlen, "malformed or unsupported .qlm");
    or_model_free(m);
    return NULL;
}

void or_model_free(or_model *m) {
    if (!m) return;
    if (m->map && m->map != MAP_FAILED) munmap(m->map, m->map_size);
    free(m->tensors);
    free(m->layers);
    free(m->x), free(m->xb), free(m->xb2), free(m->q), free(m->hb), free(m->hb2), free(m->att);
    free(m->logits), free(m->kc), free(m->vc), free(m->xq);
    free(m);
}

void or_model_dims(const or_model *m, int32_t out[7]) {
    out[0] = m->dim, out[1] = m->hidden, out[2] = m->n_layers, out[3] = m->n_heads;
    out[4] = m->n_kv_heads, out[5] = m->vocab, out[6] = m->max_seq;
}

static void mv(or_model *m, const or_tensor *W, const float *x, float *y) {
    or_matvec(W->dtype, W->data, W->ne[0], W->ne[1], x, y, m->xq);
}

/* reference src/model.c:158-191 with the per-head attention of src/model.c:127-156 */
float *or_model_forward(or_model *m, int32_t token, int32_t pos) {
    if (token < 0 || token >= m->vocab || pos < 0 || pos >= m->max_seq) return NULL;
    int64_t D = m->dim, H = m->hidden, hd = D / m->n_heads, kvd = hd * m->n_kv_heads;
    int64_t group = m->n_heads / m->n_kv_heads, S = m->max_seq;
    float scale = 1.0f / sqrtf((float)hd);
    const or_tensor *E = m->tok_embd;
    or_row_to_f32(E->dtype, E->data + (size_t)token * or_row_bytes(E->dtype, D), m->x, D);
    for (int l = 0; l < m->n_layers; l++) {
        const or_layer *L = &m->layers[l];
        float *kl = m->kc + (size_t)l * S * kvd, *vl = m->vc + (size_t)l * S * kvd;
        or_rmsnorm(m->xb, m->x, (const float *)(const void *)L->attn_norm->data, D, m->eps);
        mv(m, L->wq, m->xb, m->q);
        mv(m, L->wk, m->xb, kl + (size_t)pos * kvd);
        mv(m, L->wv, m->xb, vl + (size_t)pos * kvd);
        or_rope(m->q, m->n_heads, hd, pos, m->theta);
        or_rope(kl + (size_t)pos * kvd, m->n_kv_heads, hd, pos, m->theta);
        for (int64_t h = 0; h < m->n_heads; h++) {
            const float *qh = m->q + h * hd;
            int64_t kvh = h / group;
            for (int32_t t = 0; t <= pos; t++) m->att[t] = or_dot_f32(qh, kl + (size_t)t * kvd + kvh * hd, hd) * scale;
            or_softmax(m->att, pos + 1);
            float *out = m->xb + h * hd;
            for (int64_t i = 0; i < hd; i++) {
                float acc = 0.0f;
                for (int32_t t = 0; t <= pos; t++) acc = acc + m->att[t] * vl[(size_t)t * kvd + kvh * hd + i];
                out[i] = acc;
            }
        }
        mv(m, L->wo, m->xb, m->xb2);
        for (int64_t i = 0; i < D; i++) m->x[i] = m->x[i] + m->xb2[i];
        or_rmsnorm(m->xb, m->x, (const float *)(const void *)L->ffn_norm->data, D, m->eps);
        mv(m, L->w1, m->xb, m->hb);
        mv(m, L->w3, m->xb, m->hb2);
        or_swiglu(m->hb, m->hb2, H);
        mv(m, L->w2, m->hb, m->xb);
        for (int64_t i = 0; i < D; i++) m->x[i] = m->x[i] + m->xb[i];
    }
    or_rmsnorm(m->x, m->x, (const float *)(const void *)m->norm->data, D, m->eps);
    mv(m, m->output, m->x, m->logits);
    return m->logits;
}
