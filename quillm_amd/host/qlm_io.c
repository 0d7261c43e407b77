/* .qlm reader (mmap) and synthetic-model generator for the HIP host. C11. */
#define _GNU_SOURCE /* sincosf */
#include "qlm_io.h"

#include <fcntl.h>
#include <math.h>
#include <pthread.h>
#include <stdatomic.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

size_t qlm_row_bytes(int dtype, int64_t n) { /* reference src/quant.c:7-14 */
    int64_t nb = (n + 31) / 32;
    if (dtype == QMH_F32) return (size_t)n * 4;
    if (dtype == QMH_Q8_0) return (size_t)nb * 34;
    if (dtype == QMH_Q4_0) return (size_t)nb * 18;
    return 0;
}

/* ------------------------------------------------------------------ reader */

typedef struct {
    const uint8_t *p;
    size_t n, off;
    int bad;
} rdr;

static const uint8_t *rd_take(rdr *r, size_t k) {
    if (r->bad || k > r->n - r->off) {
        r->bad = 1;
        return NULL;
    }
    const uint8_t *s = r->p + r->off;
    r->off += k;
    return s;
}
static uint32_t rd_u32(rdr *r) {
    const uint8_t *b = rd_take(r, 4);
    return b ? (uint32_t)b[0] | (uint32_t)b[1] << 8 | (uint32_t)b[2] << 16 | (uint32_t)b[3] << 24 : 0;
}
static uint64_t rd_u64(rdr *r) {
    uint64_t lo = rd_u32(r);
    return lo | (uint64_t)rd_u32(r) << 32;
}
static int rd_name(rdr *r, char *dst, size_t cap) {
    uint32_t len = rd_u32(r);
    if (r->bad || len == 0 || len >= cap) return -1;
    const uint8_t *s = rd_take(r, len);
    if (!s || memchr(s, 0, len)) return -1;
    memcpy(dst, s, len);
    dst[len] = 0;
    return 0;
}

static int set_err(char *err, size_t errlen, const char *msg) {
    if (err && errlen) snprintf(err, errlen, "%s", msg);
    return -1;
}

int qlm_map_open(qlm_map *f, const char *path, char *err, size_t errlen) {
    memset(f, 0, sizeof *f);
    int fd = open(path, O_RDONLY);
    if (fd < 0) {
        if (err && errlen) snprintf(err, errlen, "cannot open %s", path);
        return -1;
    }
    struct stat st;
    if (fstat(fd, &st) != 0 || st.st_size <= 0) {
        close(fd);
        return set_err(err, errlen, "cannot stat file");
    }
    f->size = (size_t)st.st_size;
    void *map = mmap(NULL, f->size, PROT_READ, MAP_PRIVATE, fd, 0);
    close(fd);
    if (map == MAP_FAILED) return set_err(err, errlen, "mmap failed");
    f->map = map;
    rdr r = {f->map, f->size, 0, 0};
    const uint8_t *magic = rd_take(&r, 4);
    uint32_t ver = rd_u32(&r), n_kv = rd_u32(&r), n_t = rd_u32(&r);
    uint64_t data_off = rd_u64(&r);
    if (!magic || memcmp(magic, "QLMF", 4) || r.bad) goto bad;
    if (ver != 1) {
        qlm_map_close(f);
        return set_err(err, errlen, "unsupported version");
    }
    if (n_kv > 256 || n_t > 4096 || data_off % 64 || data_off > f->size) goto bad;
    qmh_config *c = &f->cfg;
    c->rope_theta = 10000.0f; /* defaults, reference src/model.c:46-47 */
    c->norm_eps = 1e-5f;
    static const char *keys[7] = {"llama.dim",        "llama.hidden_dim", "llama.n_layers", "llama.n_heads",
                                  "llama.n_kv_heads", "llama.vocab_size", "llama.max_seq"};
    int32_t *dst[7] = {&c->dim, &c->hidden_dim, &c->n_layers, &c->n_heads, &c->n_kv_heads, &c->vocab_size, &c->max_seq};
    int seen[9] = {0}; /* the 7 keys above, rope_theta, norm_eps */
    for (uint32_t i = 0; i < n_kv; i++) {
        char key[64];
        if (rd_name(&r, key, sizeof key)) goto bad;
        uint32_t ty = rd_u32(&r), v = 0;
        if (ty == 0 || ty == 1) v = rd_u32(&r);
        else if (ty == 2) rd_take(&r, rd_u32(&r));
        else if (ty == 3) {
            uint32_t cnt = rd_u32(&r);
            if (cnt > (f->size - r.off) / 4) goto bad;
            rd_take(&r, (size_t)cnt * 4);
        } else goto bad;
        if (r.bad) goto bad;
        /* the first entry of a key decides, as the reference's lookup returns the first match
         * (src/qlm_file.c:181-185; src/model.c:8-21): a later duplicate is ignored */
        for (int k = 0; k < 7; k++)
            if (!seen[k] && !strcmp(key, keys[k])) {
                seen[k] = 1;
                f->have[k] = ty == 0 && v != 0 && v <= (1u << 24);
                if (f->have[k]) *dst[k] = (int32_t)v;
            }
        if (!seen[7] && !strcmp(key, "llama.rope_theta")) {
            seen[7] = 1;
            if (ty == 1) memcpy(&c->rope_theta, &v, 4);
        }
        if (!seen[8] && !strcmp(key, "llama.norm_eps")) {
            seen[8] = 1;
            if (ty == 1) memcpy(&c->norm_eps, &v, 4);
        }
    }
    f->tensors = calloc(n_t ? n_t : 1, sizeof(qlm_tensor));
    if (!f->tensors) goto bad;
    f->n_tensors = n_t;
    size_t data_size = f->size - data_off;
    for (uint32_t i = 0; i < n_t; i++) {
        qlm_tensor *t = &f->tensors[i];
        if (rd_name(&r, t->name, sizeof t->name)) goto bad;
        uint32_t dt = rd_u32(&r), nd = rd_u32(&r);
        if (r.bad || !(dt == QMH_F32 || dt == QMH_Q8_0 || dt == QMH_Q4_0) || nd < 1 || nd > 4) goto bad;
        t->view.dtype = (int32_t)dt;
        t->view.ndim = (int32_t)nd;
        uint64_t nelem = 1;
        for (uint32_t d = 0; d < nd; d++) {
            uint64_t ne = rd_u64(&r);
            if (ne == 0 || ne > ((uint64_t)1 << 40) || nelem > ((uint64_t)1 << 40) / ne) goto bad;
            nelem *= ne;
            t->view.ne[d] = (int64_t)ne;
        }
        uint64_t off = rd_u64(&r);
        if (r.bad || off % 64) goto bad;
        int64_t rows = 1;
        for (uint32_t d = 0; d + 1 < nd; d++) rows *= t->view.ne[d];
        size_t bytes = (size_t)rows * qlm_row_bytes((int)dt, t->view.ne[nd - 1]);
        if (off > data_size || bytes > data_size - off) {
            qlm_map_close(f);
            return set_err(err, errlen, "tensor out of range");
        }
        t->view.data = f->map + data_off + off;
    }
    if (r.off > data_off) goto bad;
    return 0;
bad:
    qlm_map_close(f);
    return set_err(err, errlen, "malformed .qlm header");
}

void qlm_map_close(qlm_map *f) {
    if (f->map) munmap(f->map, f->size);
    free(f->tensors);
    memset(f, 0, sizeof *f);
}

const qlm_tensor *qlm_map_find(const qlm_map *f, const char *name) {
    for (uint32_t i = 0; i < f->n_tensors; i++)
        if (!strcmp(f->tensors[i].name, name)) return &f->tensors[i];
    return NULL;
}

/* ------------------------------------------------------------------ host quantizer
 * The generator stores weights exactly as the reference's quantizer would (src/quant.c:33-85):
 * d = amax/qmax in fp32, rounded to fp16 (nearest-even), codes clamp(rint(x/fp32(d))). */

static uint16_t host_f2h(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    uint32_t sign = (u >> 16) & 0x8000u, a = u & 0x7fffffffu;
    if (a > 0x7f800000u) return (uint16_t)(sign | 0x7e00u | ((a >> 13) & 0x3ffu));
    int e = (int)(a >> 23) - 127;
    if (e >= 16) return (uint16_t)(sign | 0x7c00u);
    if (e < -25) return (uint16_t)sign;
    uint32_t mant = (a & 0x7fffffu) | 0x800000u;
    int sh = e >= -14 ? 13 : 13 + (-14 - e);
    uint32_t q = mant >> sh, rem = mant & ((1u << sh) - 1u), half = 1u << (sh - 1);
    q += (rem > half || (rem == half && (q & 1u))) ? 1u : 0u;
    uint32_t res = e >= -14 ? (((uint32_t)(e + 14) << 10) + q) : q;
    return (uint16_t)(sign | res);
}

static float host_h2f(uint16_t h) {
    uint32_t sign = (uint32_t)(h >> 15) << 31, e = (h >> 10) & 31u, m = h & 1023u, bits;
    if (e == 31) bits = sign | 0x7f800000u | (m << 13);
    else if (e) bits = sign | ((e + 112u) << 23) | (m << 13);
    else {
        float v = (float)m * 0x1p-24f;
        memcpy(&bits, &v, 4);
        bits |= sign;
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

static void host_quantize_row(int dtype, const float *x, int64_t n, uint8_t *out) {
    const float qmax = dtype == QMH_Q4_0 ? 7.0f : 127.0f, qmin = dtype == QMH_Q4_0 ? -8.0f : -127.0f;
    const int bs = dtype == QMH_Q4_0 ? 18 : 34;
    for (int64_t b = 0; b < (n + 31) / 32; b++) {
        float v[32], amax = 0.0f;
        for (int i = 0; i < 32; i++) {
            int64_t k = b * 32 + i;
            v[i] = k < n ? x[k] : 0.0f;
            float a = fabsf(v[i]);
            amax = a > amax ? a : amax;
        }
        uint16_t dh = host_f2h(amax / qmax);
        float dd = host_h2f(dh);
        uint8_t *blk = out + b * bs;
        blk[0] = (uint8_t)(dh & 0xff);
        blk[1] = (uint8_t)(dh >> 8);
        int q[32];
        for (int i = 0; i < 32; i++) {
            if (dd == 0.0f) {
                q[i] = 0;
                continue;
            }
            float r = rintf(v[i] / dd);
            r = r < qmin ? qmin : r;
            r = r > qmax ? qmax : r;
            q[i] = (int)r;
        }
        if (dtype == QMH_Q8_0)
            for (int i = 0; i < 32; i++) blk[2 + i] = (uint8_t)(int8_t)q[i];
        else
            for (int j = 0; j < 16; j++) blk[2 + j] = (uint8_t)((q[2 * j] + 8) | ((q[2 * j + 1] + 8) << 4));
    }
}

/* ------------------------------------------------------------------ generator */

static uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ULL;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebULL;
    return z ^ (z >> 31);
}

/* Elements 2p and 2p+1 of tensor ti are the pair of N(0,1) variates Box-Muller makes from one
 * 64-bit hash of (seed, ti, p), scaled by 0.02: r*cos(t) and r*sin(t) in fp32. */
static void gen_pair(uint64_t base, int64_t p, float *z0, float *z1) {
    uint64_t h = mix64(base + (uint64_t)p * 0x9e3779b97f4a7c15ULL);
    float u1 = ((float)(h >> 40) + 0.5f) * 0x1p-24f, u2 = (float)(h & 0xffffffu) * 0x1p-24f;
    float r = sqrtf(-2.0f * logf(u1)), s, c;
    sincosf(6.2831853f * u2, &s, &c);
    *z0 = 0.02f * (r * c);
    *z1 = 0.02f * (r * s);
}

static uint64_t gen_base(uint64_t seed, int ti) { return mix64(seed ^ mix64((uint64_t)ti + 0x51ed2701ULL)); }

/* out[i] = value of element k0+i */
static void gen_fill(uint64_t base, int64_t k0, int64_t n, float *out) {
    int64_t i = 0;
    float a, b;
    if (n > 0 && (k0 & 1)) { /* odd start: second half of a pair */
        gen_pair(base, k0 >> 1, &a, &b);
        out[i++] = b;
    }
    for (; i + 1 < n; i += 2) gen_pair(base, (k0 + i) >> 1, &out[i], &out[i + 1]);
    if (i < n) {
        gen_pair(base, (k0 + i) >> 1, &a, &b);
        out[i] = a;
    }
}

void qmh_gen_values(uint64_t seed, int tensor_index, int64_t k0, int64_t n, float *out) {
    gen_fill(gen_base(seed, tensor_index), k0, n, out);
}

typedef struct {
    char name[64];
    int dtype, ndim;
    int64_t ne[2];
    uint64_t off;
    size_t bytes;
    int norm; /* 1-D gain: all 1.0 */
} gen_tensor;

typedef struct {
    const gen_tensor *ts;
    int nt;
    uint8_t *data;
    uint64_t seed;
    int64_t total_units;
    int64_t *unit_tensor, *unit_row0;
    atomic_llong next;
} gen_job;

#define GEN_ROWS_PER_UNIT 64

static void *gen_worker(void *arg) {
    gen_job *j = arg;
    float *buf = NULL;
    size_t cap = 0;
    for (;;) {
        long long u = atomic_fetch_add(&j->next, 1);
        if (u >= j->total_units) break;
        const gen_tensor *t = &j->ts[j->unit_tensor[u]];
        int64_t cols = t->ndim == 2 ? t->ne[1] : t->ne[0], rows = t->ndim == 2 ? t->ne[0] : 1;
        int64_t r0 = j->unit_row0[u], r1 = r0 + GEN_ROWS_PER_UNIT < rows ? r0 + GEN_ROWS_PER_UNIT : rows;
        if ((size_t)cols > cap) {
            free(buf);
            cap = (size_t)cols;
            buf = malloc(cap * sizeof(float));
            if (!buf) return (void *)1;
        }
        size_t rb = qlm_row_bytes(t->dtype, cols);
        uint64_t base = gen_base(j->seed, (int)j->unit_tensor[u]);
        for (int64_t r = r0; r < r1; r++) {
            if (t->norm)
                for (int64_t c = 0; c < cols; c++) buf[c] = 1.0f;
            else
                gen_fill(base, r * cols, cols, buf);
            uint8_t *dst = j->data + t->off + (size_t)r * rb;
            if (t->dtype == QMH_F32) memcpy(dst, buf, (size_t)cols * 4);
            else host_quantize_row(t->dtype, buf, cols, dst);
        }
    }
    free(buf);
    return NULL;
}

static void put32(uint8_t **p, uint32_t v) {
    for (int i = 0; i < 4; i++) *(*p)++ = (uint8_t)(v >> (8 * i));
}
static void put64(uint8_t **p, uint64_t v) {
    for (int i = 0; i < 8; i++) *(*p)++ = (uint8_t)(v >> (8 * i));
}
static void putname(uint8_t **p, const char *s) {
    uint32_t n = (uint32_t)strlen(s);
    put32(p, n);
    memcpy(*p, s, n);
    *p += n;
}

int qmh_gen_qlm_impl(const char *path, const qmh_config *cfg, int wtype, uint64_t seed, int n_threads, char *err,
                     size_t errlen) {
    if (!(wtype == QMH_F32 || wtype == QMH_Q8_0 || wtype == QMH_Q4_0)) return set_err(err, errlen, "bad wtype");
    if (cfg->dim <= 0 || cfg->hidden_dim <= 0 || cfg->n_layers <= 0 || cfg->n_heads <= 0 || cfg->n_kv_heads <= 0 ||
        cfg->vocab_size <= 0 || cfg->max_seq <= 0 || cfg->dim % cfg->n_heads || cfg->n_heads % cfg->n_kv_heads)
        return set_err(err, errlen, "bad config");
    const int64_t D = cfg->dim, H = cfg->hidden_dim, V = cfg->vocab_size, L = cfg->n_layers;
    const int64_t KV = D / cfg->n_heads * cfg->n_kv_heads;
    int nt = (int)(3 + 9 * L);
    gen_tensor *ts = calloc((size_t)nt, sizeof(gen_tensor));
    if (!ts) return set_err(err, errlen, "out of memory");
    int k = 0;
#define ADD2(nm, r, c)                                                                                               \
    do {                                                                                                             \
        snprintf(ts[k].name, 64, "%s", nm);                                                                          \
        ts[k].dtype = wtype, ts[k].ndim = 2, ts[k].ne[0] = r, ts[k].ne[1] = c;                                       \
        k++;                                                                                                         \
    } while (0)
#define ADD1(nm, n)                                                                                                  \
    do {                                                                                                             \
        snprintf(ts[k].name, 64, "%s", nm);                                                                          \
        ts[k].dtype = QMH_F32, ts[k].ndim = 1, ts[k].ne[0] = n, ts[k].norm = 1;                                      \
        k++;                                                                                                         \
    } while (0)
    /* tensor order of the reference's writer: tok_embd, per layer attn_norm wq wk wv wo
     * ffn_norm w1 w2 w3, then norm, output */
    ADD2("tok_embd", V, D);
    for (int64_t l = 0; l < L; l++) {
        char nm[64];
        snprintf(nm, 64, "layers.%d.attn_norm", (int)l);
        ADD1(nm, D);
        snprintf(nm, 64, "layers.%d.wq", (int)l);
        ADD2(nm, D, D);
        snprintf(nm, 64, "layers.%d.wk", (int)l);
        ADD2(nm, KV, D);
        snprintf(nm, 64, "layers.%d.wv", (int)l);
        ADD2(nm, KV, D);
        snprintf(nm, 64, "layers.%d.wo", (int)l);
        ADD2(nm, D, D);
        snprintf(nm, 64, "layers.%d.ffn_norm", (int)l);
        ADD1(nm, D);
        snprintf(nm, 64, "layers.%d.w1", (int)l);
        ADD2(nm, H, D);
        snprintf(nm, 64, "layers.%d.w2", (int)l);
        ADD2(nm, D, H);
        snprintf(nm, 64, "layers.%d.w3", (int)l);
        ADD2(nm, H, D);
    }
    ADD1("norm", D);
    ADD2("output", V, D);
#undef ADD1
#undef ADD2
    /* header */
    const char *kv_u32[7] = {"llama.dim",        "llama.hidden_dim", "llama.n_layers", "llama.n_heads",
                             "llama.n_kv_heads", "llama.vocab_size", "llama.max_seq"};
    const uint32_t kv_val[7] = {(uint32_t)cfg->dim,        (uint32_t)cfg->hidden_dim, (uint32_t)cfg->n_layers,
                                (uint32_t)cfg->n_heads,    (uint32_t)cfg->n_kv_heads, (uint32_t)cfg->vocab_size,
                                (uint32_t)cfg->max_seq};
    size_t hsz = 24 + (4 + strlen("general.name") + 4 + 4 + strlen("quillm-random"));
    for (int i = 0; i < 7; i++) hsz += 4 + strlen(kv_u32[i]) + 4 + 4;
    hsz += (4 + strlen("llama.rope_theta") + 4 + 4) + (4 + strlen("llama.norm_eps") + 4 + 4);
    uint64_t off = 0;
    for (int i = 0; i < nt; i++) {
        hsz += 4 + strlen(ts[i].name) + 8 + 8 * (size_t)ts[i].ndim + 8;
        int64_t rows = ts[i].ndim == 2 ? ts[i].ne[0] : 1, cols = ts[i].ndim == 2 ? ts[i].ne[1] : ts[i].ne[0];
        ts[i].bytes = (size_t)rows * qlm_row_bytes(ts[i].dtype, cols);
        ts[i].off = off;
        off += (ts[i].bytes + 63) / 64 * 64;
    }
    uint64_t data_off = (hsz + 63) / 64 * 64, total = data_off + off;
    int fd = open(path, O_RDWR | O_CREAT | O_TRUNC, 0644);
    if (fd < 0) {
        free(ts);
        return set_err(err, errlen, "cannot create output file");
    }
    if (ftruncate(fd, (off_t)total) != 0) {
        close(fd);
        free(ts);
        return set_err(err, errlen, "ftruncate failed (disk full?)");
    }
    uint8_t *map = mmap(NULL, total, PROT_READ | PROT_WRITE, MAP_SHARED, fd, 0);
    close(fd);
    if (map == MAP_FAILED) {
        free(ts);
        return set_err(err, errlen, "mmap of output failed");
    }
    uint8_t *p = map;
    memcpy(p, "QLMF", 4), p += 4;
    put32(&p, 1);
    put32(&p, 10);
    put32(&p, (uint32_t)nt);
    put64(&p, data_off);
    putname(&p, "general.name");
    put32(&p, 2);
    putname(&p, "quillm-random");
    for (int i = 0; i < 7; i++) {
        putname(&p, kv_u32[i]);
        put32(&p, 0);
        put32(&p, kv_val[i]);
    }
    uint32_t fb;
    putname(&p, "llama.rope_theta");
    put32(&p, 1);
    memcpy(&fb, &cfg->rope_theta, 4), put32(&p, fb);
    putname(&p, "llama.norm_eps");
    put32(&p, 1);
    memcpy(&fb, &cfg->norm_eps, 4), put32(&p, fb);
    for (int i = 0; i < nt; i++) {
        putname(&p, ts[i].name);
        put32(&p, (uint32_t)ts[i].dtype);
        put32(&p, (uint32_t)ts[i].ndim);
        for (int d = 0; d < ts[i].ndim; d++) put64(&p, (uint64_t)ts[i].ne[d]);
        put64(&p, ts[i].off);
    }
    if ((uint64_t)(p - map) != hsz) {
        munmap(map, total);
        free(ts);
        return set_err(err, errlen, "internal: header size mismatch");
    }
    memset(p, 0, data_off - hsz);
    /* data: units of 64 rows, handed out to threads */
    int64_t units = 0;
    for (int i = 0; i < nt; i++) units += ((ts[i].ndim == 2 ? ts[i].ne[0] : 1) + GEN_ROWS_PER_UNIT - 1) / GEN_ROWS_PER_UNIT;
    gen_job job = {ts, nt, map + data_off, seed, units, malloc(sizeof(int64_t) * (size_t)units),
                   malloc(sizeof(int64_t) * (size_t)units), 0};
    if (!job.unit_tensor || !job.unit_row0) {
        munmap(map, total);
        free(ts), free(job.unit_tensor), free(job.unit_row0);
        return set_err(err, errlen, "out of memory");
    }
    int64_t u = 0;
    for (int i = 0; i < nt; i++) {
        int64_t rows = ts[i].ndim == 2 ? ts[i].ne[0] : 1;
        for (int64_t r = 0; r < rows; r += GEN_ROWS_PER_UNIT) job.unit_tensor[u] = i, job.unit_row0[u++] = r;
    }
    atomic_init(&job.next, 0);
    if (n_threads < 1) n_threads = 1;
    if (n_threads > 256) n_threads = 256;
    pthread_t th[256];
    int started = 0, failed = 0;
    for (int i = 1; i < n_threads; i++)
        if (pthread_create(&th[started], NULL, gen_worker, &job) == 0) started++;
    if (gen_worker(&job)) failed = 1;
    for (int i = 0; i < started; i++) {
        void *rv;
        pthread_join(th[i], &rv);
        if (rv) failed = 1;
    }
    /* padding between tensors is zero already (fresh file) */
    munmap(map, total);
    free(ts), free(job.unit_tensor), free(job.unit_row0);
    return failed ? set_err(err, errlen, "generator worker failed") : 0;
}
