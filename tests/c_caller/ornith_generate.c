/* ornith_generate.c - a C11 program that drives the engine through its C ABI
 * (include/ornith_hip.h) the way a caller of the reference's rmodel API does
 * (src/ornith_rforward.h:24-130: rmodel_load, rmodel_arch,
 * rmodel_session_new / _eval / _logits / _generate / _free): load a GGUF,
 * open a session, evaluate a prompt, generate greedily, print the tokens.
 *
 * usage: ornith_generate <model.gguf> <n_generate> <prompt token>...
 * prints "arch ...", "argmax <id>" (the prompt logits' greedy token),
 * "tokens <id> <id> ..." and "pos <n>"; exit status 0, or 1 with the
 * library's message on stderr. A session one position short of the prompt
 * must be refused with ORNITH_HIP_ERR_UNSUPPORTED (the reference's capacity
 * error), which the program checks before the real run. */
#include <stdio.h>
#include <stdlib.h>

#include "ornith_hip.h"

static int fail(const char *what, int st) {
    fprintf(stderr, "%s: status %d: %s\n", what, st, ornith_hip_last_error());
    return 1;
}

int main(int argc, char **argv) {
    if (argc < 4) {
        fprintf(stderr, "usage: %s <model.gguf> <n_generate> <prompt token>...\n", argv[0]);
        return 2;
    }
    const int n_gen = atoi(argv[2]), n_prompt = argc - 3;
    int32_t *prompt = malloc(sizeof(int32_t) * (size_t)n_prompt);
    int32_t *out = malloc(sizeof(int32_t) * (size_t)(n_gen > 0 ? n_gen : 1));
    if (!prompt || !out) return 1;
    for (int i = 0; i < n_prompt; i++) prompt[i] = (int32_t)atoi(argv[3 + i]);

    ornith_hip_ctx *ctx = NULL;
    ornith_hip_model *m = NULL;
    ornith_hip_session *s = NULL;
    int st;
    if ((st = ornith_hip_init(0, &ctx)) != ORNITH_HIP_OK) return fail("init", st);
    if ((st = ornith_hip_model_load(ctx, argv[1], &m)) != ORNITH_HIP_OK) return fail("model_load", st);
    ornith_hip_arch a;
    if ((st = ornith_hip_model_arch(m, &a)) != ORNITH_HIP_OK) return fail("model_arch", st);
    printf("arch hidden %d layers %d vocab %d heads %d/%d experts %d top %d\n", (int)a.hidden,
           (int)a.n_layers, (int)a.vocab, (int)a.nh, (int)a.nkv, (int)a.ne, (int)a.top_k);

    /* the capacity error path: a session one position short of the prompt */
    if ((st = ornith_hip_session_new(m, n_prompt - 1 > 0 ? n_prompt - 1 : 1, &s)) != ORNITH_HIP_OK)
        return fail("session_new", st);
    st = ornith_hip_session_eval(s, prompt, n_prompt);
    if (n_prompt > 1 && st != ORNITH_HIP_ERR_UNSUPPORTED) {
        fprintf(stderr, "capacity: expected status %d, got %d\n", ORNITH_HIP_ERR_UNSUPPORTED, st);
        return 1;
    }
    ornith_hip_session_free(s);
    s = NULL;

    if ((st = ornith_hip_session_new(m, n_prompt + n_gen + 1, &s)) != ORNITH_HIP_OK)
        return fail("session_new", st);
    if ((st = ornith_hip_session_eval(s, prompt, n_prompt)) != ORNITH_HIP_OK) return fail("session_eval", st);
    float *logits = malloc(sizeof(float) * (size_t)a.vocab);
    if (!logits) return 1;
    if ((st = ornith_hip_session_logits(s, logits)) != ORNITH_HIP_OK) return fail("session_logits", st);
    int best = 0;
    for (int i = 1; i < a.vocab; i++)
        if (logits[i] > logits[best]) best = i;
    printf("argmax %d\n", best);
    int n_out = 0;
    if ((st = ornith_hip_session_generate(s, n_gen, out, &n_out)) != ORNITH_HIP_OK)
        return fail("session_generate", st);
    printf("tokens");
    for (int i = 0; i < n_out; i++) printf(" %d", (int)out[i]);
    printf("\npos %d\n", ornith_hip_session_pos(s));

    ornith_hip_session_free(s);
    ornith_hip_model_free(m);
    ornith_hip_free(ctx);
    free(logits);
    free(out);
    free(prompt);
    return 0;
}
