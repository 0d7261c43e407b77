/* ref_driver: a harness around the compiled REFERENCE (its public API only: model.h,
 * sampler.h, kernels.h). TEST INFRASTRUCTURE ONLY -- it is the "reference" CPU path that
 * parity tests and bench.py's cpu_baseline leg run; nothing in quillm_amd/ uses it.
 *
 *   ref_driver MODEL.qlm --prompt FILE [--gen G] [--isa scalar|avx2|avx512] [--threads N]
 *              [--max-seq S] [--logits FILE] [--warm]
 *
 * Prompt: P token ids from FILE (whitespace separated). Runs the reference's only prompt
 * method, P sequential qm_model_forward calls (reference src/main.c:127-130), then G greedy
 * steps timed like reference bench/bench.c:143-149: next = argmax(forward(tok, pos)), EOS not
 * treated as a stop. --logits writes every position's logits (P+G rows of vocab floats).
 * Prints one JSON object.
 */
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

#include "kernels.h"
#include "model.h"
#include "sampler.h"

static double now_s(void) {
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return (double)ts.tv_sec + (double)ts.tv_nsec * 1e-9;
}

int main(int argc, char **argv) {
    if (argc < 2) {
        fprintf(stderr, "usage: ref_driver MODEL.qlm --prompt FILE [--gen G] [--isa I] [--threads N] [--max-seq S] [--logits F] [--warm]\n");
        return 2;
    }
    const char *path = argv[1], *prompt_file = NULL, *isa = NULL, *logits_file = NULL;
    int gen = 0, threads = 1, max_seq = 0, warm = 0;
    for (int i = 2; i < argc; i++) {
        const char *a = argv[i];
        int has = i + 1 < argc;
        if (!strcmp(a, "--prompt") && has) prompt_file = argv[++i];
        else if (!strcmp(a, "--gen") && has) gen = atoi(argv[++i]);
        else if (!strcmp(a, "--isa") && has) isa = argv[++i];
        else if (!strcmp(a, "--threads") && has) threads = atoi(argv[++i]);
        else if (!strcmp(a, "--max-seq") && has) max_seq = atoi(argv[++i]);
        else if (!strcmp(a, "--logits") && has) logits_file = argv[++i];
        else if (!strcmp(a, "--warm")) warm = 1;
        else {
            fprintf(stderr, "bad argument %s\n", a);
            return 2;
        }
    }
    if (isa) {
        int lvl = qm_isa_from_name(isa);
        if (lvl < 0 || qm_kernels_select((qm_isa)lvl) != 0) {
            fprintf(stderr, "ISA %s not available\n", isa);
            return 1;
        }
    }
    int cap = 1 << 16, n_prompt = 0;
    int32_t *prompt = malloc(sizeof(int32_t) * (size_t)cap);
    FILE *pf = prompt_file ? fopen(prompt_file, "r") : NULL;
    if (!pf) {
        fprintf(stderr, "cannot read prompt file\n");
        return 1;
    }
    while (n_prompt < cap && fscanf(pf, "%d", &prompt[n_prompt]) == 1) n_prompt++;
    fclose(pf);
    if (n_prompt < 1) {
        fprintf(stderr, "empty prompt\n");
        return 1;
    }
    qm_model m;
    char err[256];
    double tl = now_s();
    if (qm_model_load(&m, path, threads, max_seq, err, sizeof err) != 0) {
        fprintf(stderr, "load: %s\n", err);
        return 1;
    }
    tl = now_s() - tl;
    int V = m.cfg.vocab_size;
    if (n_prompt + gen > m.cfg.max_seq) {
        fprintf(stderr, "prompt+gen exceeds max_seq %d\n", m.cfg.max_seq);
        return 1;
    }
    FILE *lf = logits_file ? fopen(logits_file, "wb") : NULL;
    if (warm) { /* one untimed pass over a few positions: pages the mmap'd weights in */
        for (int i = 0; i < n_prompt && i < 2; i++) qm_model_forward(&m, prompt[i], i);
    }
    float *logits = NULL;
    double t0 = now_s();
    for (int i = 0; i < n_prompt; i++) {
        logits = qm_model_forward(&m, prompt[i], i);
        if (lf) fwrite(logits, sizeof(float), (size_t)V, lf);
    }
    double t_prompt = now_s() - t0;
    int32_t *toks = malloc(sizeof(int32_t) * (size_t)(gen + 1));
    toks[0] = qm_argmax(logits, V);
    double t1 = now_s();
    for (int g = 0; g < gen; g++) {
        logits = qm_model_forward(&m, toks[g], n_prompt + g);
        if (lf) fwrite(logits, sizeof(float), (size_t)V, lf);
        toks[g + 1] = qm_argmax(logits, V);
    }
    double t_gen = now_s() - t1;
    if (lf) fclose(lf);
    printf("{\"isa\": \"%s\", \"threads\": %d, \"max_seq\": %d, \"n_prompt\": %d, \"n_gen\": %d, \"load_s\": %.6f, "
           "\"prompt_s\": %.6f, \"decode_s\": %.6f, \"prompt_tok_s\": %.4f, \"decode_tok_s\": %.4f, \"tokens\": [",
           qm_isa_name(qm_kernels_active()->isa), m.n_threads, m.cfg.max_seq, n_prompt, gen, tl, t_prompt, t_gen,
           n_prompt / (t_prompt > 0 ? t_prompt : 1e-9), gen / (t_gen > 0 ? t_gen : 1e-9));
    for (int g = 0; g <= gen; g++) printf("%s%d", g ? ", " : "", toks[g]);
    printf("]}\n");
    free(toks);
    free(prompt);
    qm_model_free(&m);
    return 0;
}
