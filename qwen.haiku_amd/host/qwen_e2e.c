/*
 * qwen_e2e.c -- end-to-end driver of qwen.haiku's forward pass on a
 * random-init Qwen3.5-0.8B-shaped model.
 *
 * Built twice from this one file, with the reference's own sources and
 * flags (slm/Makefile:13-17):
 *   - QK_E2E_GPU defined: qk_seam.c is included first, so every quantized
 *     matmul of the model runs through libqk on the GPU (the drop-in);
 *   - otherwise: the reference unchanged (its CPU SIMD matmuls).
 * Everything else (embedding dequant, RMSNorm, rope, attention, the
 * Gated DeltaNet recurrence and its chunked prefill, SiLU) is the
 * reference's host code in both builds, compiled identically, so the two
 * token streams are identical exactly when every matmul result is.
 *
 * Model: the reference's hybrid layout (slm/qwen.c:174-252; types of the
 * unsloth Q4_K_M mix, docs/DESIGN.md:96-119): 24 layers, hidden 1024,
 * FFN 3584, vocab 248320 (Q6_K token embedding tied to the LM head),
 * Gated DeltaNet layers with softmax attention every 4th layer
 * (8 query heads / 2 KV heads of dim 256, output gate), linear attention
 * 16 heads of 128, conv kernel 4. Weights are seeded random blocks scaled
 * so every projection keeps activations O(1): quant scales and mins are
 * chosen so the dequantised weights have mean ~0 and standard deviation
 * ~1/sqrt(k); norm weights 1 +- 0.02; ssm_a negative; small conv1d and
 * dt bias.
 *
 * Workload (mirrors slm_generate_raw, slm/slm.c:237-358, with greedy
 * sampling and no repetition penalty): a seeded random prompt of P tokens
 * through slm_forward_batch (chunked prefill), then G steps of
 * slm_forward_step starting from the last prompt token at position P,
 * each picking sample_argmax (slm/model.c:401) of the logits.
 *
 * Output: one JSON line on stdout with the token stream, prefill and
 * decode tok/s, and non-degeneracy figures; progress lines on stderr.
 *
 * GGUF round trip: --write-gguf PATH also writes the random model as a
 * GGUF v3 file (gguf_write.c: the qwen35 config keys slm_load_config
 * reads, slm/qwen.c:59-160; a synthetic vocabulary of distinct strings for
 * tokenizer_load, slm/tokenizer.c:216-275; every tensor under the names
 * slm_load_weights resolves, slm/qwen.c:174-252). --gguf PATH loads a
 * model through the reference's own slm_model_load (slm/model.c:1130) in
 * place of building one; the prompt comes from its own seeded stream, so
 * both modes run the same workload.
 *
 * Decode path of the GPU build (--decode): "chain" (default) runs each
 * step through qk_decode.c, the residual stream and the FFN resident on
 * the GPU and the greedy pick fused into the LM head; "seam" runs the
 * reference's slm_forward_step unchanged, every matmul a round trip
 * through the seam. Both report their host synchronisations per token.
 *
 * Prefill path of the GPU build (--prefill): "layer" (default) runs
 * qk_prefill.c, the reference's batched pass with each DeltaNet layer's
 * chunk loop as one GPU call; "seam" runs the reference's
 * slm_forward_batch unchanged, one GPU call per head and chunk. The JSON
 * line reports the prefill seconds spent inside GPU calls.
 *
 * --sample SEED (non-zero) replaces the greedy pick with the reference's
 * default sampler chain (slm_sampler_defaults, slm/sampler.c:22-31):
 * rng_seed(SEED) and a history holding the prompt, as slm_generate_raw
 * does (slm/slm.c:251-325). The CPU build and --decode seam call the
 * reference's sample_with on the host; --decode chain calls hip_sample on
 * the device logits.
 *
 * Usage: qwen_e2e [--prompt P] [--gen G] [--seed S] [--layers L]
 *                 [--write-gguf PATH | --gguf PATH] [--decode chain|seam]
 *                 [--prefill layer|seam] [--sample SEED]
 */
#if defined(QK_E2E_GPU)
#include "qk_seam.c"
#endif
#include "qwen.c"
#include "sampler.c"
#include "gguf_write.c"
#if defined(QK_E2E_GPU)
#include "qk_decode.c"
#include "qk_prefill.c"
#endif

#include <time.h>

/* ---- deterministic random numbers (splitmix64) ------------------------- */
static uint64_t e2e_state;

static uint64_t e2e_u64(void) {
    uint64_t z = (e2e_state += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

static double e2e_unif(void) { return (double)(e2e_u64() >> 11) * (1.0 / 9007199254740992.0); }

static int32_t e2e_int(int32_t lo, int32_t hi) { return lo + (int32_t)(e2e_u64() % (uint64_t)(hi - lo + 1)); }

/* The prompt's own stream: the same tokens whether the weights are drawn
 * here or loaded from a file. */
static uint64_t e2e_prompt_state;

static int32_t e2e_prompt_token(int32_t vocab) {
    uint64_t z = (e2e_prompt_state += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    z ^= z >> 31;
    return (int32_t)(z % (uint64_t)vocab);
}

static uint16_t e2e_f16(double v) {
    _Float16 h = (_Float16)(float)v;
    uint16_t u;
    memcpy(&u, &h, 2);
    return u;
}

/* ---- random quantized blocks ------------------------------------------- */
/* Packing of 8 six-bit scales and mins into 12 bytes: the inverse of
 * q4k_get_scale_min (simd/quants.h:215-224). */
static void e2e_pack_scales(uint8_t *s, const uint8_t *sc, const uint8_t *mn) {
    for (int j = 0; j < 4; j++) {
        s[j] = (uint8_t)((sc[j] & 63) | ((sc[j + 4] >> 4) << 6));
        s[j + 4] = (uint8_t)((mn[j] & 63) | ((mn[j + 4] >> 4) << 6));
        s[j + 8] = (uint8_t)((sc[j + 4] & 15) | ((mn[j + 4] & 15) << 4));
    }
}

/* d jitter in [0.75, 1.25) so blocks differ in scale. */
static double e2e_jit(void) { return 0.75 + 0.5 * e2e_unif(); }

/* Q4_K: w = d*sc*q - dmin*m with dmin = d, sc in [1,8], m = round(7.5 sc),
 * q uniform in [0,15]: mean ~0, std ~ d*4.5*4.6. */
static void e2e_q4k(q4k_block *b, int64_t n, double sigma) {
    for (int64_t i = 0; i < n; i++) {
        uint8_t sc[8], mn[8];
        for (int j = 0; j < 8; j++) {
            sc[j] = (uint8_t)e2e_int(1, 8);
            mn[j] = (uint8_t)(7.5 * sc[j] + 0.5);
        }
        uint16_t d = e2e_f16(sigma / 20.7 * e2e_jit());
        memcpy(&b[i].d, &d, 2);
        memcpy(&b[i].dmin, &d, 2);
        e2e_pack_scales(b[i].scales, sc, mn);
        for (int j = 0; j < QK_K / 2; j++) b[i].qs[j] = (uint8_t)e2e_u64();
    }
}

/* Q5_K: q in [0,31], sc in [1,4], m = round(15.5 sc). */
static void e2e_q5k(q5k_block *b, int64_t n, double sigma) {
    for (int64_t i = 0; i < n; i++) {
        uint8_t sc[8], mn[8];
        for (int j = 0; j < 8; j++) {
            sc[j] = (uint8_t)e2e_int(1, 4);
            mn[j] = (uint8_t)(15.5 * sc[j] + 0.5);
        }
        uint16_t d = e2e_f16(sigma / 23.0 * e2e_jit());
        memcpy(&b[i].d, &d, 2);
        memcpy(&b[i].dmin, &d, 2);
        e2e_pack_scales(b[i].scales, sc, mn);
        for (int j = 0; j < QK_K / 8; j++) b[i].qh[j] = (uint8_t)e2e_u64();
        for (int j = 0; j < QK_K / 2; j++) b[i].qs[j] = (uint8_t)e2e_u64();
    }
}

/* Q6_K: w = d*sc*(u6-32), sc int8 in [-32,31]. */
static void e2e_q6k(q6k_block *b, int64_t n, double sigma) {
    for (int64_t i = 0; i < n; i++) {
        for (int j = 0; j < QK_K / 2; j++) b[i].ql[j] = (uint8_t)e2e_u64();
        for (int j = 0; j < QK_K / 4; j++) b[i].qh[j] = (uint8_t)e2e_u64();
        for (int j = 0; j < QK_K / 16; j++) b[i].scales[j] = (int8_t)e2e_int(-32, 31);
        uint16_t d = e2e_f16(sigma / 340.0 * e2e_jit());
        memcpy(&b[i].d, &d, 2);
    }
}

/* Q8_0: w = d*q, q in [-127,127]. */
static void e2e_q8_0(q8_0_block *b, int64_t n, double sigma) {
    for (int64_t i = 0; i < n; i++) {
        uint16_t d = e2e_f16(sigma / 73.0 * e2e_jit());
        memcpy(&b[i].d, &d, 2);
        for (int j = 0; j < QK8_0; j++) b[i].qs[j] = (int8_t)e2e_int(-127, 127);
    }
}

/* When writing a GGUF: every tensor built is also recorded under its
 * slm_load_weights name. */
static struct gw *e2e_gw;

static void e2e_set(struct slm_tensor *t, const char *name, const void *data, int32_t type, int64_t n0,
                    int64_t n1, uint64_t bytes) {
    t->data = data;
    t->type = type;
    t->n_dims = n1 > 1 ? 2 : 1;
    t->shape[0] = n0;
    t->shape[1] = n1;
    t->shape[2] = 1;
    t->shape[3] = 1;
    if (e2e_gw) {
        const uint64_t shape[2] = {(uint64_t)n0, (uint64_t)n1};
        gw_tensor(e2e_gw, name, (uint32_t)type, (uint32_t)t->n_dims, shape, data, bytes);
    }
}

/* Quantized weight (GGUF shape (k, out_f)): out_f rows of k elements. */
static void e2e_mat(struct slm_tensor *t, const char *name, int32_t type, int64_t k, int64_t out_f, double scale) {
    const double sigma = scale / sqrt((double)k);
    void *p = NULL;
    uint64_t bytes = 0;
    switch (type) {
        case GGUF_TT_Q4_K:
            p = oom(calloc((size_t)(out_f * k / QK_K), sizeof(q4k_block)));
            e2e_q4k(p, out_f * k / QK_K, sigma);
            bytes = (uint64_t)(out_f * k / QK_K) * sizeof(q4k_block);
            break;
        case GGUF_TT_Q5_K:
            p = oom(calloc((size_t)(out_f * k / QK_K), sizeof(q5k_block)));
            e2e_q5k(p, out_f * k / QK_K, sigma);
            bytes = (uint64_t)(out_f * k / QK_K) * sizeof(q5k_block);
            break;
        case GGUF_TT_Q6_K:
            p = oom(calloc((size_t)(out_f * k / QK_K), sizeof(q6k_block)));
            e2e_q6k(p, out_f * k / QK_K, sigma);
            bytes = (uint64_t)(out_f * k / QK_K) * sizeof(q6k_block);
            break;
        default:
            p = oom(calloc((size_t)(out_f * k / QK8_0), sizeof(q8_0_block)));
            e2e_q8_0(p, out_f * k / QK8_0, sigma);
            bytes = (uint64_t)(out_f * k / QK8_0) * sizeof(q8_0_block);
            break;
    }
    e2e_set(t, name, p, type, k, out_f, bytes);
#if defined(QK_E2E_GPU)
    qk_seam_register(p, type, k, out_f);
#endif
}

static void e2e_vec(struct slm_tensor *t, const char *name, int64_t n0, int64_t n1, double base, double spread) {
    float *p = (float *)oom(calloc((size_t)(n0 * n1), sizeof(float)));
    for (int64_t i = 0; i < n0 * n1; i++) p[i] = (float)(base + spread * (2.0 * e2e_unif() - 1.0));
    e2e_set(t, name, p, GGUF_TT_F32, n0, n1, (uint64_t)(n0 * n1) * sizeof(float));
}

/* Vocabulary strings of the written GGUF: distinct, none of them a chat
 * special, so tokenizer_load finds no specials and eot_id stays -1 as in
 * the built model. */
static size_t e2e_token_name(uint64_t i, char *buf, size_t cap) {
    return (size_t)snprintf(buf, cap, "<t%llu>", (unsigned long long)i);
}

/* The qwen35 keys slm_load_config reads (slm/qwen.c:59-160). */
static void e2e_write_config(struct gw *w, const struct slm_config *c) {
    gw_kv_str(w, "general.architecture", "qwen35");
    gw_kv_u32(w, "general.alignment", 32);
    gw_kv_u32(w, "qwen35.embedding_length", (uint32_t)c->hidden_dim);
    gw_kv_u32(w, "qwen35.block_count", (uint32_t)c->n_layers);
    gw_kv_u32(w, "qwen35.attention.head_count", (uint32_t)c->n_heads);
    gw_kv_u32(w, "qwen35.attention.head_count_kv", (uint32_t)c->n_kv_heads);
    gw_kv_u32(w, "qwen35.feed_forward_length", (uint32_t)c->ffn_dim);
    gw_kv_u32(w, "qwen35.context_length", 4096);
    gw_kv_f32(w, "qwen35.rope.freq_base", c->rope_theta);
    gw_kv_f32(w, "qwen35.attention.layer_norm_rms_epsilon", c->norm_eps);
    gw_kv_u32(w, "qwen35.attention.key_length", (uint32_t)c->head_dim);
    gw_kv_u32(w, "qwen35.rope.dimension_count", (uint32_t)c->rope_dim);
    gw_kv_i32_array(w, "qwen35.rope.dimension_sections", c->rope_sections, 4);
    gw_kv_u32(w, "qwen35.full_attention_interval", (uint32_t)c->full_attn_interval);
    gw_kv_u32(w, "qwen35.ssm.group_count", (uint32_t)c->linear_n_heads);
    gw_kv_u32(w, "qwen35.ssm.state_size", (uint32_t)c->linear_k_head_dim);
    gw_kv_u32(w, "qwen35.ssm.conv_kernel", (uint32_t)c->linear_conv_kernel);
    gw_kv_str_array(w, "tokenizer.ggml.tokens", (uint64_t)c->vocab_size, e2e_token_name);
}

static double e2e_now(void) {
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return (double)ts.tv_sec + 1e-9 * (double)ts.tv_nsec;
}

int main(int argc, char **argv) {
    int32_t n_prompt = 512, n_gen = 256, n_layers = 24;
    uint64_t seed = 0, sample_seed = 0;
    const char *write_path = NULL, *load_path = NULL, *decode_mode = "chain", *prefill_mode = "layer";
    for (int i = 1; i + 1 < argc; i += 2) {
        if (strcmp(argv[i], "--prompt") == 0) n_prompt = atoi(argv[i + 1]);
        else if (strcmp(argv[i], "--gen") == 0) n_gen = atoi(argv[i + 1]);
        else if (strcmp(argv[i], "--seed") == 0) seed = (uint64_t)strtoull(argv[i + 1], NULL, 10);
        else if (strcmp(argv[i], "--layers") == 0) n_layers = atoi(argv[i + 1]);
        else if (strcmp(argv[i], "--write-gguf") == 0) write_path = argv[i + 1];
        else if (strcmp(argv[i], "--gguf") == 0) load_path = argv[i + 1];
        else if (strcmp(argv[i], "--decode") == 0) decode_mode = argv[i + 1];
        else if (strcmp(argv[i], "--prefill") == 0) prefill_mode = argv[i + 1];
        else if (strcmp(argv[i], "--sample") == 0) sample_seed = (uint64_t)strtoull(argv[i + 1], NULL, 10);
    }
    const int chain = strcmp(decode_mode, "chain") == 0, layer_prefill = strcmp(prefill_mode, "layer") == 0;
    if (n_prompt < 2 || n_gen < 1 || n_layers < 1 || (write_path && load_path) ||
        (!chain && strcmp(decode_mode, "seam") != 0) || (!layer_prefill && strcmp(prefill_mode, "seam") != 0)) {
        fprintf(stderr, "usage: %s [--prompt P>=2] [--gen G>=1] [--seed S] [--layers L>=1] "
                        "[--write-gguf PATH | --gguf PATH] [--decode chain|seam] [--prefill layer|seam] "
                        "[--sample SEED]\n", argv[0]);
        return 2;
    }
    simd_init();
    e2e_state = seed * 0x2545F4914F6CDD1Dull + 1;
    e2e_prompt_state = seed * 0x2545F4914F6CDD1Dull + 2;

    struct slm_config cfg;
    memset(&cfg, 0, sizeof(cfg));
    cfg.n_layers = n_layers;
    cfg.n_heads = 8;
    cfg.n_kv_heads = 2;
    cfg.head_dim = 256;
    cfg.hidden_dim = 1024;
    cfg.ffn_dim = 3584;
    cfg.vocab_size = 248320;
    cfg.max_position = n_prompt + n_gen + 1;
    cfg.rope_theta = 10000000.0f;
    cfg.rope_dim = 64;
    cfg.norm_eps = 1e-6f;
    cfg.bos_id = -1;
    cfg.eos_id = -1;
    cfg.eot_id = -1;
    cfg.attn_output_gate = 1;
    cfg.is_hybrid = 1;
    cfg.full_attn_interval = 4;
    cfg.linear_n_heads = 16;
    cfg.linear_k_head_dim = 128;
    cfg.linear_v_head_dim = 128;
    cfg.linear_conv_kernel = 4;
    cfg.rope_sections[0] = 11;
    cfg.rope_sections[1] = 11;
    cfg.rope_sections[2] = 10;
    cfg.rope_sections[3] = 0;
    const int64_t H = cfg.hidden_dim, F = cfg.ffn_dim, V = cfg.vocab_size;
    const int64_t QKV = 2 * 16 * 128 + 16 * 128, INNER = 16 * 128;

    double tb = e2e_now();
    struct slm_model *m = NULL;
    struct gw gw;
    if (load_path) {
        /* the reference's loader: config keys, tensor names, tokenizer */
        m = slm_model_load(load_path);
        if (!slm_model_loaded(m)) {
            fprintf(stderr, "[e2e] slm_model_load(%s): %s\n", load_path, slm_model_error(m));
            return 1;
        }
        if (m->cfg.n_layers != n_layers || m->cfg.vocab_size != cfg.vocab_size) {
            fprintf(stderr, "[e2e] %s holds %d layers / vocab %d; expected %d / %d\n", load_path,
                    m->cfg.n_layers, m->cfg.vocab_size, n_layers, cfg.vocab_size);
            return 1;
        }
        /* the run's KV-cache length and ids, as the built model sets them
           (the forward pass reads neither bos nor eos) */
        m->cfg.max_position = cfg.max_position;
        m->cfg.bos_id = cfg.bos_id;
        m->cfg.eos_id = cfg.eos_id;
    } else {
        if (write_path) {
            gw_init(&gw);
            e2e_write_config(&gw, &cfg);
            e2e_gw = &gw;
        }
        m = (struct slm_model *)oom(calloc(1, sizeof(struct slm_model)));
        m->cfg = cfg;
        struct slm_weights *W = &m->W;
        e2e_mat(&W->tok_embd, "token_embd.weight", GGUF_TT_Q6_K, H, V, 1.5);
        W->output = W->tok_embd;                               /* tied (slm/qwen.c:182-183) */
        e2e_vec(&W->output_norm, "output_norm.weight", H, 1, 1.0, 0.02);
        W->layers = (struct slm_layer *)oom(calloc((size_t)n_layers, sizeof(struct slm_layer)));
        char nm[96];
#define NM(fmt) (snprintf(nm, sizeof(nm), fmt, L), nm)
        for (int32_t L = 0; L < n_layers; L++) {
            struct slm_layer *Lw = &W->layers[L];
            Lw->is_ssm = (L % cfg.full_attn_interval) != cfg.full_attn_interval - 1;
            e2e_vec(&Lw->attn_norm, NM("blk.%d.attn_norm.weight"), H, 1, 1.0, 0.02);
            e2e_vec(&Lw->ffn_norm, NM("blk.%d.post_attention_norm.weight"), H, 1, 1.0, 0.02);
            e2e_mat(&Lw->ffn_gate, NM("blk.%d.ffn_gate.weight"), GGUF_TT_Q4_K, H, F, 1.0);
            e2e_mat(&Lw->ffn_up, NM("blk.%d.ffn_up.weight"), GGUF_TT_Q4_K, H, F, 1.0);
            e2e_mat(&Lw->ffn_down, NM("blk.%d.ffn_down.weight"), GGUF_TT_Q6_K, F, H, 0.5);
            if (Lw->is_ssm) {
                e2e_mat(&Lw->attn_qkv, NM("blk.%d.attn_qkv.weight"), GGUF_TT_Q5_K, H, QKV, 1.0);
                e2e_mat(&Lw->attn_gate, NM("blk.%d.attn_gate.weight"), GGUF_TT_Q4_K, H, INNER, 1.0);
                e2e_vec(&Lw->ssm_a, NM("blk.%d.ssm_a"), 16, 1, -1.25, 0.75);
                e2e_mat(&Lw->ssm_alpha, NM("blk.%d.ssm_alpha.weight"), GGUF_TT_Q8_0, H, 16, 1.0);
                e2e_mat(&Lw->ssm_beta, NM("blk.%d.ssm_beta.weight"), GGUF_TT_Q8_0, H, 16, 1.0);
                e2e_vec(&Lw->ssm_conv1d, NM("blk.%d.ssm_conv1d.weight"), 4, QKV, 0.0, 0.5);
                e2e_vec(&Lw->ssm_dt_bias, NM("blk.%d.ssm_dt.bias"), 16, 1, 0.0, 0.1);
                e2e_vec(&Lw->ssm_norm, NM("blk.%d.ssm_norm.weight"), 128, 1, 1.0, 0.02);
                e2e_mat(&Lw->ssm_out, NM("blk.%d.ssm_out.weight"), GGUF_TT_Q5_K, INNER, H, 0.5);
            } else {
                e2e_mat(&Lw->attn_q, NM("blk.%d.attn_q.weight"), GGUF_TT_Q5_K, H, 2 * 8 * 256, 1.0);
                e2e_mat(&Lw->attn_k, NM("blk.%d.attn_k.weight"), GGUF_TT_Q4_K, H, 2 * 256, 1.0);
                e2e_mat(&Lw->attn_v, NM("blk.%d.attn_v.weight"), GGUF_TT_Q6_K, H, 2 * 256, 1.0);
                e2e_vec(&Lw->attn_q_norm, NM("blk.%d.attn_q_norm.weight"), 256, 1, 1.0, 0.02);
                e2e_vec(&Lw->attn_k_norm, NM("blk.%d.attn_k_norm.weight"), 256, 1, 1.0, 0.02);
                e2e_mat(&Lw->attn_out, NM("blk.%d.attn_output.weight"), GGUF_TT_Q4_K, 8 * 256, H, 0.5);
            }
        }
#undef NM
        m->loaded = 1;
        if (write_path) {
            uint64_t total = 0;
            if (gw_write(&gw, write_path, &total) != 0) {
                fprintf(stderr, "[e2e] writing %s failed\n", write_path);
                return 1;
            }
            fprintf(stderr, "[e2e] wrote %s: %llu bytes, %llu tensors\n", write_path, (unsigned long long)total,
                    (unsigned long long)gw.n_t);
            gw_free(&gw);
            e2e_gw = NULL;
        }
    }
    struct slm_ctx *c = slm_ctx_create(m);
    int32_t *prompt = (int32_t *)oom(calloc((size_t)n_prompt, sizeof(int32_t)));
    for (int32_t i = 0; i < n_prompt; i++) prompt[i] = e2e_prompt_token((int32_t)V);
    int32_t *toks = (int32_t *)oom(calloc((size_t)n_gen, sizeof(int32_t)));
    fprintf(stderr, "[e2e] %s: model %s in %.2f s (%d layers), prefill %d tokens\n",
#if defined(QK_E2E_GPU)
            "gpu",
#else
            "cpu",
#endif
            load_path ? "loaded" : "built", e2e_now() - tb, n_layers, n_prompt);

    /* prefill (slm/slm.c:278-283) */
    double t0 = e2e_now();
#if defined(QK_E2E_GPU)
    struct tensor *logits = layer_prefill ? qk_forward_batch(c, prompt, n_prompt, 0)
                                          : slm_forward_batch(c, prompt, n_prompt, 0);
#else
    (void)layer_prefill;
    struct tensor *logits = slm_forward_batch(c, prompt, n_prompt, 0);
#endif
    /* the prefill's last-token logits, for the stream comparison */
    double pl_min = logits->data[0], pl_max = logits->data[0], pl_sum = 0;
    for (int64_t i = 0; i < (int64_t)cfg.vocab_size; i++) {
        const double v = logits->data[i];
        pl_min = v < pl_min ? v : pl_min;
        pl_max = v > pl_max ? v : pl_max;
        pl_sum += v;
    }
    int32_t pos = n_prompt;
    double t1 = e2e_now();
    double pf_mm = 0.0, pf_dn = 0.0;   /* prefill seconds inside the GPU matmul / DeltaNet calls */
#if defined(QK_E2E_GPU)
    pf_mm = qk_seam_matmul_s;
    pf_dn = qk_seam_deltanet_s + qk_prefill_layer_calls;
#endif
    fprintf(stderr, "[e2e] prefill %.3f s\n", t1 - t0);

    /* decode (slm/slm.c:307-358): the first step re-feeds the last prompt token */
    int32_t last = prompt[n_prompt - 1];
    int64_t nonfinite = 0;
    double lmin = 0, lmax = 0, lsum = 0, lsq = 0;
    const int64_t nvocab = cfg.vocab_size;
    float *lbuf = (float *)oom(malloc((size_t)nvocab * sizeof(float)));
    long long syncs0 = 0, hits0 = 0, miss0 = 0;
    /* sampling state (slm/slm.c:251-263) */
    struct slm_sampler sp = slm_sampler_defaults();
    const struct slm_sampler *spp = sample_seed ? &sp : NULL;
    int32_t *history = (int32_t *)oom(calloc((size_t)(n_prompt + n_gen + 1), sizeof(int32_t)));
    int32_t hist_n = 0;
    for (int32_t i = 0; i < n_prompt; i++) history[hist_n++] = prompt[i];
    if (sample_seed) rng_seed(&c->rng, sample_seed);
#if defined(QK_E2E_GPU)
    qk_dec D;
    if (chain) {
        qk_dec_init(&D, m);
        if (sample_seed) qk_dec_sampling(&D, &c->rng, history, hist_n, n_prompt + n_gen + 1);
    }
    syncs0 = qk_seam_gpu_calls;
    hits0 = qk_seam_pf_hits;
    miss0 = qk_seam_pf_misses;
#else
    (void)chain;
#endif
    const double td = e2e_now();       /* decode clock: after the device step's one-time setup */
    for (int32_t g = 0; g < n_gen; g++) {
        const int stats = g == 0 || g == n_gen - 1;
        int32_t next;
        const float *lv = NULL;
#if defined(QK_E2E_GPU)
        if (chain) {
            next = qk_decode_step(c, &D, last, pos, stats ? lbuf : NULL, spp);
            lv = lbuf;
        } else
#endif
        {
            logits = slm_forward_step(c, last, pos);
            lv = logits->data;
            if (spp && stats) {            /* sample_with penalizes in place: keep the raw logits */
                memcpy(lbuf, lv, (size_t)nvocab * sizeof(float));
                lv = lbuf;
            }
            next = spp ? sample_with(logits, spp, &c->rng, history, hist_n) : sample_argmax(logits);
        }
        history[hist_n++] = next;
        if (stats) {
            lmin = lmax = lv[0];
            lsum = lsq = 0;
            for (int64_t i = 0; i < nvocab; i++) {
                float v = lv[i];
                if (!(v == v) || v > 3e38f || v < -3e38f) nonfinite++;
                lmin = v < lmin ? v : lmin;
                lmax = v > lmax ? v : lmax;
                lsum += v;
                lsq += (double)v * v;
            }
        }
        toks[g] = next;
        last = next;
        pos++;
        if ((g + 1) % 32 == 0) fprintf(stderr, "[e2e] decoded %d / %d\n", g + 1, n_gen);
    }
    double t2 = e2e_now();
    /* host synchronisations with the GPU per decoded token: every seam
       matmul that reached the GPU, plus the device step's own waits */
    double syncs_per_tok = 0, pf_hits = 0, pf_misses = 0;
#if defined(QK_E2E_GPU)
    syncs_per_tok = (double)(qk_seam_gpu_calls - syncs0 + (chain ? D.syncs : 0)) / n_gen;
    pf_hits = (double)(qk_seam_pf_hits - hits0);
    pf_misses = (double)(qk_seam_pf_misses - miss0);
#else
    (void)syncs0; (void)hits0; (void)miss0;
#endif

    int32_t distinct = 0;
    for (int32_t i = 0; i < n_gen; i++) {
        int32_t seen = 0;
        for (int32_t j = 0; j < i && !seen; j++) seen = toks[j] == toks[i];
        distinct += !seen;
    }
    const double nv = (double)cfg.vocab_size;
    printf("{\"mode\": \"%s\", \"source\": \"%s\", \"tier\": \"%s\", \"layers\": %d, \"prompt\": %d, \"gen\": %d, \"seed\": %llu, "
           "\"prefill_s\": %.6f, \"prefill_gpu_matmul_s\": %.6f, \"prefill_gpu_deltanet_s\": %.6f, "
           "\"prefill_path\": \"%s\", \"prefill_logits\": {\"min\": %.9g, \"max\": %.9g, \"sum\": %.17g}, "
           "\"decode_s\": %.6f, \"prefill_tok_s\": %.3f, \"decode_tok_s\": %.3f, "
           "\"decode_path\": \"%s\", \"sampler\": \"%s\", \"host_syncs_per_token\": %.2f, \"prefetch_hits\": %.0f, \"prefetch_misses\": %.0f, "
           "\"distinct_tokens\": %d, \"nonfinite_logits\": %lld, \"last_logits\": {\"min\": %.6g, \"max\": %.6g, "
           "\"mean\": %.6g, \"std\": %.6g}, \"tokens\": [",
#if defined(QK_E2E_GPU)
           "gpu",
#else
           "cpu",
#endif
           load_path ? "gguf" : "built", simd_dispatch_label(), n_layers, n_prompt, n_gen, (unsigned long long)seed, t1 - t0, pf_mm, pf_dn,
#if defined(QK_E2E_GPU)
           layer_prefill ? "gpu-layer" : "gpu-seam",
#else
           "cpu",
#endif
           pl_min, pl_max, pl_sum, t2 - td,
           n_prompt / (t1 - t0), n_gen / (t2 - td),
#if defined(QK_E2E_GPU)
           chain ? "gpu-chain" : "gpu-seam",
#else
           "cpu",
#endif
           spp ? "slm_sampler_defaults" : "greedy", syncs_per_tok, pf_hits, pf_misses, distinct, (long long)nonfinite, lmin, lmax, lsum / nv,
           sqrt(lsq / nv - (lsum / nv) * (lsum / nv)));
    for (int32_t i = 0; i < n_gen; i++) printf("%s%d", i ? ", " : "", toks[i]);
    printf("]}\n");
    fflush(stdout);
#if defined(QK_E2E_GPU)
    if (chain) qk_dec_free(&D);
#endif
    slm_ctx_destroy(c);
    return nonfinite ? 1 : 0;
}
