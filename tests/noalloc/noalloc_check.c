/* noalloc_check: the device path's restatement of the reference's tests/test_noalloc.c -- TEST
 * INFRASTRUCTURE. The reference's forward performs no heap allocation (src/model.h:35), which its test
 * proves by counting malloc/calloc/realloc/aligned_alloc. Here the process's allocator itself is
 * replaced (glibc allows a program to define malloc and friends; these forward to __libc_*), so every
 * heap allocation in the process is counted, the HIP runtime's included, without preloading anything.
 *
 *   noalloc_check MODEL.qlm MAX_SEQ
 *
 * After the model and a sampler are created and one warm-up call of each entry point has run, counts
 * the allocations of MAX_SEQ qmh_model_forward calls (the reference test's loop: each token the argmax
 * of the previous logits), then of qmh_model_greedy and qmh_model_sample over the same positions.
 * Prints one line per phase: every allocation in the process, and those libqmhip.so made itself; each
 * allocation is attributed (backtrace, dladdr) to the library function and, when the HIP runtime
 * allocated, the HIP entry point that the library called.
 *
 * Then qmh_sample_noalloc, the entry point for callers that cannot allocate: after one warm-up call,
 * 32 calls at a vocabulary above 8192 (the multi-workgroup path) and 32 at one below it, counted like
 * the phases above, with the device's free memory (hipMemGetInfo) read before and after. Last, the
 * same draw captured in a HIP graph (the caller it is for) and replayed 8 times, eager draws of a
 * sampler object between the replays: each replay's token and rng state against the eager draw's. */
#define _GNU_SOURCE
#include <dlfcn.h>
#include <execinfo.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <hip/hip_runtime_api.h>

#include "../../include/qmhip.h"

void *__libc_malloc(size_t);
void *__libc_calloc(size_t, size_t);
void *__libc_realloc(void *, size_t);
void *__libc_memalign(size_t, size_t);
void __libc_free(void *);

static volatile int g_on;
static volatile long g_count, g_own;
static _Thread_local int g_in;  /* inside note(): backtrace and dladdr may allocate themselves */

/* where an allocation comes from: the first frame (walking out from the allocator) that is neither
 * the C/C++ runtime nor this program. In libqmhip.so the library allocated itself (g_own); else the
 * HIP runtime did, inside the HIP API entry that the outermost libqmhip.so frame called */
#define NSITE 16
static struct {
    char who[96];
    long n;
} g_sites[NSITE];

static int in_lib(const char *f, const char *name) { return f && strstr(f, name) != NULL; }

static void attribute(void) {
    void *fr[48];
    int n = backtrace(fr, 48);
    const char *api = "?", *caller = "?";
    int own = 0, found = 0;
    for (int i = 2; i < n && !found; i++) {
        Dl_info di;
        if (!dladdr(fr[i], &di)) continue;
        if (in_lib(di.dli_fname, "libqmhip")) {
            /* the first foreign frame is ours: the library allocated */
            own = 1;
            caller = di.dli_sname ? di.dli_sname : "?";
            found = 1;
        } else if (!in_lib(di.dli_fname, "libc.so") && !in_lib(di.dli_fname, "libstdc++") &&
                   !in_lib(di.dli_fname, "noalloc_check")) {
            /* runtime frame: find the libqmhip.so frame that entered the runtime, and the entry */
            for (int j = i + 1; j < n; j++) {
                Dl_info dj;
                if (dladdr(fr[j], &dj) && in_lib(dj.dli_fname, "libqmhip")) {
                    caller = dj.dli_sname ? dj.dli_sname : "?";
                    Dl_info de;
                    if (dladdr(fr[j - 1], &de) && de.dli_sname) api = de.dli_sname;
                    break;
                }
            }
            found = 1;
        }
    }
    if (own) __atomic_fetch_add(&g_own, 1, __ATOMIC_RELAXED);
    char who[96];
    snprintf(who, sizeof who, "%s%s <- %s", own ? "LIBRARY " : "", api, caller);
    for (int k = 0; k < NSITE; k++) {
        if (g_sites[k].n == 0) {
            snprintf(g_sites[k].who, sizeof g_sites[k].who, "%s", who);
            g_sites[k].n = 1;
            return;
        }
        if (strcmp(g_sites[k].who, who) == 0) {
            g_sites[k].n++;
            return;
        }
    }
}

static void note(void *ra) {
    (void)ra;
    if (!g_on || g_in) return;
    g_in = 1;
    __atomic_fetch_add(&g_count, 1, __ATOMIC_RELAXED);
    attribute();
    g_in = 0;
}
void *malloc(size_t n) {
    note(__builtin_return_address(0));
    return __libc_malloc(n);
}
void *calloc(size_t a, size_t b) {
    note(__builtin_return_address(0));
    return __libc_calloc(a, b);
}
void *realloc(void *p, size_t n) {
    note(__builtin_return_address(0));
    return __libc_realloc(p, n);
}
void *aligned_alloc(size_t a, size_t n) {
    note(__builtin_return_address(0));
    return __libc_memalign(a, n);
}
void *memalign(size_t a, size_t n) {
    note(__builtin_return_address(0));
    return __libc_memalign(a, n);
}
int posix_memalign(void **out, size_t a, size_t n) {
    note(__builtin_return_address(0));
    void *p = __libc_memalign(a, n);
    if (!p) return 12; /* ENOMEM */
    *out = p;
    return 0;
}
void free(void *p) { __libc_free(p); }

static int argmax(const float *x, int n) {
    int b = 0;
    for (int i = 1; i < n; i++)
        if (x[i] > x[b]) b = i;
    return b;
}

static void begin(void) {
    g_count = 0;
    g_own = 0;
    memset(g_sites, 0, sizeof g_sites);
    g_on = 1;
}

/* one line per phase: all allocations, then those the library made itself, then by site */
static long end(const char *phase, int steps) {
    g_on = 0;
    long n = g_count;
    printf("%s: %d steps, %ld heap allocations, %ld by the library\n", phase, steps, n, (long)g_own);
    for (int k = 0; k < NSITE && g_sites[k].n; k++) printf("  %6ld  %s\n", g_sites[k].n, g_sites[k].who);
    fflush(stdout);
    return g_own;
}

int main(int argc, char **argv) {
    if (argc < 3) {
        fprintf(stderr, "usage: noalloc_check MODEL.qlm MAX_SEQ\n");
        return 2;
    }
    const int S = atoi(argv[2]);
    if (qmh_init(0) != 0) {
        fprintf(stderr, "init: %s\n", qmh_last_error());
        return 1;
    }
    void *warm[4];
    backtrace(warm, 4); /* its first call loads the unwinder (allocates) */
    begin(); /* the reference test's sanity check: counting is live */
    qmh_model *m = qmh_model_load(argv[1], S);
    const long at_load = g_count;
    end("load (expected to allocate)", 0);
    if (!m) {
        fprintf(stderr, "load: %s\n", qmh_last_error());
        return 1;
    }
    if (at_load == 0) {
        fprintf(stderr, "counting inactive?\n");
        return 1;
    }
    const int V = qmh_model_config(m)->vocab_size;
    qmh_sampler *s = qmh_sampler_create(V, 0.8f, 0, 0.95f, 42);
    int32_t *out = malloc(sizeof(int32_t) * (size_t)S);
    if (!s || !out) {
        fprintf(stderr, "sampler: %s\n", qmh_last_error());
        return 1;
    }
    /* warm-up: one call of each entry point (first launches, graph and stream setup) */
    const float *lg = qmh_model_forward(m, 0, 0);
    if (!lg || qmh_model_greedy(m, argmax(lg, V), 1, 2, out) || qmh_model_sample(m, s, 3, 1, 2, out)) {
        fprintf(stderr, "warm-up: %s\n", qmh_last_error());
        return 1;
    }
    long total = 0;
    begin();
    int tok = 0;
    for (int pos = 0; pos < S; pos++) {
        lg = qmh_model_forward(m, tok, pos);
        if (!lg) {
            g_on = 0;
            fprintf(stderr, "forward: %s\n", qmh_last_error());
            return 1;
        }
        tok = argmax(lg, V);
    }
    total += end("qmh_model_forward", S);
    begin();
    int rc = qmh_model_greedy(m, 0, 0, S, out);
    total += end("qmh_model_greedy", S);
    begin();
    rc |= qmh_model_sample(m, s, 0, 0, S, out);
    total += end("qmh_model_sample", S);
    if (rc) {
        fprintf(stderr, "decode: %s\n", qmh_last_error());
        return 1;
    }
    qmh_sampler_free(s);
    qmh_model_free(m);
    free(out);
    printf("hot-loop heap allocations made by the library: %ld\n", total);

    /* qmh_sample_noalloc: logits of a fixed pseudo-random pattern, vocabularies 32000 and 4000 */
    enum { NV = 32000, NS = 4000 };
    float *hl = malloc(sizeof(float) * NV);
    float *dl = qmh_dev_alloc(sizeof(float) * NV);
    uint64_t *drng = qmh_dev_alloc(sizeof(uint64_t)), *drng2 = qmh_dev_alloc(sizeof(uint64_t));
    int32_t *dout = qmh_dev_alloc(sizeof(int32_t)), *dout2 = qmh_dev_alloc(sizeof(int32_t));
    if (!hl || !dl || !drng || !drng2 || !dout || !dout2) {
        fprintf(stderr, "noalloc buffers: %s\n", qmh_last_error());
        return 1;
    }
    uint64_t z = 0x2545f4914f6cdd1dull;
    for (int i = 0; i < NV; i++) {
        z = z * 6364136223846793005ull + 1442695040888963407ull;
        hl[i] = (float)((int64_t)(z >> 40) - (1 << 23)) * 0x1p-20f;  /* about [-8, 8) */
    }
    const uint64_t seed0 = 0x9e3779b97f4a7c15ull;
    if (qmh_memcpy_h2d(dl, hl, sizeof(float) * NV) || qmh_memcpy_h2d(drng, &seed0, sizeof seed0)) {
        fprintf(stderr, "noalloc setup: %s\n", qmh_last_error());
        return 1;
    }
    if (qmh_sample_noalloc(dl, NV, 0.8f, 0, 0.95f, drng, dout, NULL) ||
        qmh_sample_noalloc(dl, NS, 0.8f, 0, 0.95f, drng, dout, NULL) || qmh_sync()) {
        fprintf(stderr, "noalloc warm-up: %s\n", qmh_last_error());
        return 1;
    }
    size_t free0 = 0, free1 = 0, tot = 0;
    if (hipMemGetInfo(&free0, &tot) != hipSuccess) return 1;
    begin();
    rc = 0;
    for (int k = 0; k < 32 && rc == 0; k++) rc = qmh_sample_noalloc(dl, NV, 0.8f, 0, 0.95f, drng, dout, NULL);
    for (int k = 0; k < 32 && rc == 0; k++) rc = qmh_sample_noalloc(dl, NS, 0.8f, 0, 0.95f, drng, dout, NULL);
    rc |= qmh_sync();
    const long own_na = end("qmh_sample_noalloc", 64);
    if (rc || hipMemGetInfo(&free1, &tot) != hipSuccess) {
        fprintf(stderr, "noalloc calls: %s\n", qmh_last_error());
        return 1;
    }
    printf("qmh_sample_noalloc device free bytes: before %zu after %zu (%s)\n", free0, free1,
           free0 == free1 ? "unchanged" : "CHANGED");

    /* the draw under graph capture, replayed; eager draws of a sampler object between the replays */
    qmh_sampler *ref = qmh_sampler_create(NV, 0.8f, 0, 0.95f, 12345);
    uint64_t r0 = 0;
    hipStream_t st = NULL;
    hipGraph_t g = NULL;
    hipGraphExec_t ge = NULL;
    if (!ref || qmh_sampler_rng(ref, &r0) || qmh_memcpy_h2d(drng2, &r0, sizeof r0) || hipStreamCreate(&st) != hipSuccess ||
        hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal) != hipSuccess) {
        fprintf(stderr, "graph setup: %s\n", qmh_last_error());
        return 1;
    }
    rc = qmh_sample_noalloc(dl, NV, 0.8f, 0, 0.95f, drng2, dout2, st);
    if (hipStreamEndCapture(st, &g) != hipSuccess || rc || hipGraphInstantiate(&ge, g, NULL, NULL, 0) != hipSuccess) {
        fprintf(stderr, "graph capture failed (rc %d): %s\n", rc, qmh_last_error());
        return 1;
    }
    int bad = 0;
    for (int k = 0; k < 8; k++) {
        int32_t tg = -1, te = -1;
        uint64_t rg = 0, re = 0;
        if (hipGraphLaunch(ge, st) != hipSuccess || hipStreamSynchronize(st) != hipSuccess) return 1;
        if (qmh_memcpy_d2h(&tg, dout2, sizeof tg) || qmh_memcpy_d2h(&rg, drng2, sizeof rg)) return 1;
        te = qmh_sample_sync(ref, dl);
        if (te < 0 || qmh_sampler_rng(ref, &re)) return 1;
        printf("graph replay %d: token %d rng %016llx, eager %d rng %016llx%s\n", k, tg, (unsigned long long)rg, te,
               (unsigned long long)re, tg == te && rg == re ? "" : "  MISMATCH");
        bad += tg != te || rg != re;
    }
    hipGraphExecDestroy(ge);
    hipGraphDestroy(g);
    hipStreamDestroy(st);
    qmh_sampler_free(ref);
    printf("graph replays matching the eager draws: %d of 8\n", 8 - bad);
    fflush(stdout);
    return own_na || free0 != free1 || bad ? 3 : 0;
}
