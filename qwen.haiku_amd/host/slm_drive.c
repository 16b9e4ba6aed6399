/*
 * slm_drive.c -- the reference's own generation loop on token ids.
 *
 * This translation unit is the reference's slm/slm.c (its TU root,
 * slm/Makefile:52-87) exactly as a maintainer builds it after the
 * one-line change of INTEGRATION.md: with QK_DRIVE_GPU, qk_seam.c comes
 * first, so every quantized matmul and every chunked DeltaNet step of the
 * model runs on the GPU; without it, the unchanged reference (the CPU
 * twin, built under oracle/_ref/). slm_generate_raw (slm/slm.c:237-358)
 * is static, so this file includes slm.c and calls it from the same
 * unit: the prompt's prefill (slm_forward_step per token, or
 * slm_forward_batch with LLM_USE_FORWARD_BATCH set, slm/slm.c:271-293),
 * the repetition history, rng_seed, the min_new eos/eot masking and its
 * restore, sample_with, the stop ids and the token callback are all the
 * reference's code. The generated ids come from the reference's own
 * token trace (ctrl.trace_tokens, slm/slm.c:337-339) on stderr.
 *
 * The model is a GGUF file written by qwen_e2e --write-gguf, loaded by
 * the reference's slm_model_load (slm/model.c:1130).
 *
 * Usage: slm_drive --gguf PATH [--prompt P] [--gen G] [--seed S]
 *                  [--min-new M] [--sample SEED] [--batch]
 * Prints one JSON line on stdout: the prompt length, the generated count,
 * and the reference's own prefill and decode timings (c->t_prefill_s,
 * c->t_gen_s).
 */
#if defined(QK_DRIVE_GPU)
#include "qk_seam.c"
#endif
#include "slm.c"

static int drive_piece(const char *utf8, void *user) {
    (void)utf8;
    (void)user;
    return 0;
}

/* splitmix64 for the prompt ids, so the CPU and GPU builds feed the same */
static uint64_t drive_state;
static uint64_t drive_next(void) {
    uint64_t z = (drive_state += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

int main(int argc, char **argv) {
    const char *path = NULL;
    int32_t n_prompt = 64, n_gen = 32, min_new = 0, batch = 0;
    uint64_t seed = 0, sample_seed = 0;
    for (int i = 1; i < argc; i++) {
        if (strcmp(argv[i], "--batch") == 0) batch = 1;
        else if (i + 1 >= argc) break;
        else if (strcmp(argv[i], "--gguf") == 0) path = argv[++i];
        else if (strcmp(argv[i], "--prompt") == 0) n_prompt = atoi(argv[++i]);
        else if (strcmp(argv[i], "--gen") == 0) n_gen = atoi(argv[++i]);
        else if (strcmp(argv[i], "--seed") == 0) seed = (uint64_t)strtoull(argv[++i], NULL, 10);
        else if (strcmp(argv[i], "--min-new") == 0) min_new = atoi(argv[++i]);
        else if (strcmp(argv[i], "--sample") == 0) sample_seed = (uint64_t)strtoull(argv[++i], NULL, 10);
    }
    if (!path || n_prompt < 2 || n_gen < 1 || min_new < 0) {
        fprintf(stderr, "usage: %s --gguf PATH [--prompt P>=2] [--gen G>=1] [--seed S] [--min-new M] "
                        "[--sample SEED] [--batch]\n", argv[0]);
        return 2;
    }
    /* slm_generate_raw reads this once, on its first call */
    if (batch) setenv("LLM_USE_FORWARD_BATCH", "1", 1);
    else unsetenv("LLM_USE_FORWARD_BATCH");
    struct slm_model *m = slm_model_load(path);
    if (!slm_model_loaded(m)) {
        fprintf(stderr, "[drive] loading %s failed: %s\n", path, slm_model_error(m));
        return 1;
    }
    struct slm_ctx *c = slm_ctx_create(m);
    c->ctrl.trace_tokens = true;
    const int32_t vocab = slm_vocab_size(c);
    drive_state = seed * 0x2545F4914F6CDD1Dull + 3;
    int32_t *prompt = (int32_t *)oom(calloc((size_t)n_prompt, sizeof(int32_t)));
    for (int32_t i = 0; i < n_prompt; i++) prompt[i] = (int32_t)(drive_next() % (uint64_t)vocab);
    /* greedy with no repetition penalty, or the reference's default chain */
    struct slm_sampler sp = slm_sampler_defaults();
    if (sample_seed == 0) {
        sp.temperature = 0.0f;
        sp.repetition_penalty = 1.0f;
    }
    fprintf(stderr, "[drive] %s: %d prompt tokens, up to %d new (%s, %s prefill)\n",
#if defined(QK_DRIVE_GPU)
            "gpu",
#else
            "cpu",
#endif
            n_prompt, n_gen, sample_seed ? "sampled" : "greedy", batch ? "batch" : "per-token");
    fflush(stderr);
    const int generated = slm_generate_raw(c, prompt, n_prompt, n_gen, min_new, &sp,
                                           sample_seed ? sample_seed : 1, drive_piece, NULL, NULL, NULL);
    fflush(stderr);
    printf("{\"prompt\": %d, \"generated\": %d, \"prefill_s\": %.6f, \"decode_s\": %.6f, "
           "\"prefill_tok_s\": %.3f, \"decode_tok_s\": %.3f}\n",
           n_prompt, generated, c->t_prefill_s, c->t_gen_s, c->t_prefill_s > 0 ? n_prompt / c->t_prefill_s : 0.0,
           c->t_gen_s > 0 ? generated / c->t_gen_s : 0.0);
    free(prompt);
    slm_ctx_destroy(c);
    slm_model_unload(m);
    return 0;
}
