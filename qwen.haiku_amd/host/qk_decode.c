/*
 * qk_decode.c -- one decode step of the hybrid Qwen3.5 forward pass with
 * the residual stream resident on the GPU.
 *
 * Included by qwen_e2e.c in its GPU build, after the reference's qwen.c
 * (so it calls the reference's own mixers) and after qk_seam.c (whose
 * matmul bodies and prefetch table it uses). It follows slm_forward_step
 * (slm/qwen.c:874-985) step for step; what changes is where each step
 * runs:
 *
 *   embedding   device: Q6_K dequant of the token's row of the tied
 *               table (slm/qwen.c:891-906) into the residual stream h;
 *   per layer   device: h = h + ffn_out of the layer before, x = its
 *               attn_norm (Q8_K too), and the mixer's in-projections
 *               (SSM: attn_qkv, attn_gate, ssm_beta, ssm_alpha,
 *               slm/qwen.c:339-356; attention: attn_q, attn_k, attn_v,
 *               slm/model.c:792-794) as one grouped GEMV launch;
 *               host, synchronisation 1: h, x and the projections come
 *               back and the reference's mixer (slm_forward_ssm,
 *               slm/qwen.c:318, or slm_forward_attn, slm/model.c:766) runs
 *               on the host. It normalizes h itself and asks for its
 *               in-projections; the seam answers those from the
 *               prefetched results, after checking that its input equals
 *               x bit for bit. Its out-projection goes through the seam
 *               (synchronisation 2);
 *               device: h = h + mix, x = ffn_norm(h) as Q8_K, gate/up
 *               grouped GEMV, silu(gate) * up as Q8_K, down GEMV -> ffn_out
 *               (slm/qwen.c:932-962);
 *   head        device: h = h + ffn_out, output_norm as Q8_K, the Q6_K LM
 *               head with the greedy pick (slm/qwen.c:966-976 then
 *               sample_argmax, slm/model.c:401-412); the token id comes
 *               back (the logits only when asked for).
 *
 * Every step is bit-exact, so the token stream is the reference's. Host
 * synchronisations per token: two per layer plus one.
 */
#include <hip/hip_runtime_api.h>

#define QK_DEC_MAX_PROJ 4

/* One in-projection's output: on the device and its pinned host copy,
 * which the seam's prefetch table points at. */
typedef struct {
    float *y_dev;
    float *y_host;
} qk_dec_proj;

typedef struct {
    hipStream_t s;
    int64_t hidden, ffn, vocab;
    int32_t n_layers;
    float eps;
    float *h, *mix, *xn, *gate, *up, *act, *ffn_out, *logits;   /* device */
    void *xq, *aq;                                              /* device Q8_K rows */
    int32_t *am;                                                /* device argmax */
    float **attn_norm, **ffn_norm, *out_norm;                   /* device fp32 weights */
    float *h_host, *xn_host, *mix_host;                         /* pinned */
    int32_t *am_host;
    qk_dec_proj proj[QK_DEC_MAX_PROJ];
    long long syncs;
    /* sampling (slm_generate_raw, slm/slm.c:255-325): the rng's two words
       and the repetition history (prompt, then every pick), on the device */
    uint64_t *rng;
    int32_t *hist;
    int32_t hist_n, hist_cap;
} qk_dec;

static void qk_dec_ck(hipError_t e, const char *what) {
    if (e != hipSuccess) {
        fprintf(stderr, "qk_decode: %s: %s\n", what, hipGetErrorString(e));
        abort();
    }
}

static void qk_dec_lib(int rc, const char *what) {
    if (rc != QK_OK) {
        fprintf(stderr, "qk_decode: %s failed (%d): %s\n", what, rc, hip_qk_last_error());
        abort();
    }
}

static const void *qk_dec_weight(const struct slm_tensor *t) {
    qk_seam_register(t->data, t->type, t->shape[0], t->shape[1]);
    const void *d = hip_qk_device_weight(t->data);
    if (!d) {
        fprintf(stderr, "qk_decode: weight not on the device\n");
        abort();
    }
    return d;
}

static float *qk_dec_vec(const struct slm_tensor *t, int64_t n) {
    assert(t->type == GGUF_TT_F32 && t->shape[0] == n);
    float *d = NULL;
    qk_dec_ck(hipMalloc((void **)&d, (size_t)n * sizeof(float)), "hipMalloc(norm)");
    qk_dec_ck(hipMemcpy(d, t->data, (size_t)n * sizeof(float), hipMemcpyHostToDevice), "upload norm");
    return d;
}

static void *qk_dec_alloc(size_t bytes) {
    void *p = NULL;
    qk_dec_ck(hipMalloc(&p, bytes), "hipMalloc");
    return p;
}

static void *qk_dec_pinned(size_t bytes) {
    void *p = NULL;
    qk_dec_ck(hipHostMalloc(&p, bytes, 0), "hipHostMalloc");
    return p;
}

/* Device buffers and weights for model m: every quantized weight the
 * step reads is uploaded here (the seam keeps the copies), the F32 norm
 * weights are copied once. */
static void qk_dec_init(qk_dec *D, const struct slm_model *m) {
    memset(D, 0, sizeof(*D));
    qk_seam_init();
    const struct slm_config *cfg = &m->cfg;
    D->hidden = cfg->hidden_dim;
    D->ffn = cfg->ffn_dim;
    D->vocab = cfg->vocab_size;
    D->n_layers = cfg->n_layers;
    D->eps = cfg->norm_eps;
    if (m->W.output.type != GGUF_TT_Q6_K || m->W.tok_embd.type != GGUF_TT_Q6_K || D->hidden % QK_K ||
        D->ffn % QK_K) {
        fprintf(stderr, "qk_decode: needs Q6_K embedding / output and 256-multiple widths\n");
        abort();
    }
    qk_dec_ck(hipStreamCreate(&D->s), "hipStreamCreate");
    int64_t widest = D->ffn;                        /* the largest in-projection output */
    for (int32_t L = 0; L < cfg->n_layers; L++) {
        const struct slm_layer *Lw = &m->W.layers[L];
        const struct slm_tensor *ts[] = {&Lw->attn_qkv, &Lw->attn_gate, &Lw->ssm_beta, &Lw->ssm_alpha,
                                         &Lw->attn_q, &Lw->attn_k, &Lw->attn_v};
        for (int i = 0; i < 7; i++)
            if (ts[i]->data && ts[i]->shape[1] > widest) widest = ts[i]->shape[1];
    }
    const size_t H = (size_t)D->hidden, F = (size_t)D->ffn;
    D->h = qk_dec_alloc(H * 4);
    D->mix = qk_dec_alloc(H * 4);
    D->xn = qk_dec_alloc(H * 4);
    D->gate = qk_dec_alloc(F * 4);
    D->up = qk_dec_alloc(F * 4);
    D->act = qk_dec_alloc(F * 4);
    D->ffn_out = qk_dec_alloc(H * 4);
    D->logits = qk_dec_alloc((size_t)D->vocab * 4);
    D->xq = qk_dec_alloc(H / QK_K * 292);             /* Q8_K rows: 292 bytes per 256 */
    D->aq = qk_dec_alloc(F / QK_K * 292);
    D->am = qk_dec_alloc(sizeof(int32_t));
    D->h_host = qk_dec_pinned(H * 4);
    D->xn_host = qk_dec_pinned(H * 4);
    D->mix_host = qk_dec_pinned(H * 4);
    D->am_host = qk_dec_pinned(sizeof(int32_t));
    for (int i = 0; i < QK_DEC_MAX_PROJ; i++) {
        D->proj[i].y_dev = qk_dec_alloc((size_t)widest * 4);
        D->proj[i].y_host = qk_dec_pinned((size_t)widest * 4);
    }
    D->attn_norm = calloc((size_t)cfg->n_layers, sizeof(float *));
    D->ffn_norm = calloc((size_t)cfg->n_layers, sizeof(float *));
    for (int32_t L = 0; L < cfg->n_layers; L++) {
        const struct slm_layer *Lw = &m->W.layers[L];
        D->attn_norm[L] = qk_dec_vec(&Lw->attn_norm, D->hidden);
        D->ffn_norm[L] = qk_dec_vec(&Lw->ffn_norm, D->hidden);
        qk_dec_weight(&Lw->ffn_gate);
        qk_dec_weight(&Lw->ffn_up);
        qk_dec_weight(&Lw->ffn_down);
    }
    D->out_norm = qk_dec_vec(&m->W.output_norm, D->hidden);
    qk_dec_weight(&m->W.output);
}

/* Everything qk_dec_init and qk_dec_sampling allocated; the weights stay
 * with the seam's registry. */
static void qk_dec_free(qk_dec *D) {
    if (!D->s) return;
    qk_dec_ck(hipStreamSynchronize(D->s), "hipStreamSynchronize");
    void *dev[] = {D->h, D->mix, D->xn, D->gate, D->up, D->act, D->ffn_out, D->logits, D->xq, D->aq, D->am,
                   D->out_norm, D->rng, D->hist};
    for (size_t i = 0; i < sizeof(dev) / sizeof(dev[0]); i++)
        if (dev[i]) qk_dec_ck(hipFree(dev[i]), "hipFree");
    void *pin[] = {D->h_host, D->xn_host, D->mix_host, D->am_host};
    for (size_t i = 0; i < sizeof(pin) / sizeof(pin[0]); i++)
        if (pin[i]) qk_dec_ck(hipHostFree(pin[i]), "hipHostFree");
    for (int i = 0; i < QK_DEC_MAX_PROJ; i++) {
        if (D->proj[i].y_dev) qk_dec_ck(hipFree(D->proj[i].y_dev), "hipFree");
        if (D->proj[i].y_host) qk_dec_ck(hipHostFree(D->proj[i].y_host), "hipHostFree");
    }
    for (int32_t L = 0; D->attn_norm && D->ffn_norm && L < D->n_layers; L++) {
        qk_dec_ck(hipFree(D->attn_norm[L]), "hipFree");
        qk_dec_ck(hipFree(D->ffn_norm[L]), "hipFree");
    }
    free(D->attn_norm);
    free(D->ffn_norm);
    qk_dec_ck(hipStreamDestroy(D->s), "hipStreamDestroy");
    memset(D, 0, sizeof(*D));
}

/* Sampled decoding from the reference's rng state and a history holding
 * the prompt (slm/slm.c:251-263); room for cap ids in all. */
static void qk_dec_sampling(qk_dec *D, const struct rng *r, const int32_t *prompt, int32_t n, int32_t cap) {
    uint64_t st[2] = {r->s0, r->s1};
    D->rng = qk_dec_alloc(sizeof(st));
    D->hist = qk_dec_alloc((size_t)cap * sizeof(int32_t));
    qk_dec_ck(hipMemcpy(D->rng, st, sizeof(st), hipMemcpyHostToDevice), "upload rng");
    qk_dec_ck(hipMemcpy(D->hist, prompt, (size_t)n * sizeof(int32_t), hipMemcpyHostToDevice), "upload history");
    D->hist_n = n;
    D->hist_cap = cap;
}

/* One grouped launch of n GEMVs over the normalized row: from its Q8_K
 * copy when every weight is a K-quant, else from the fp32 row (each
 * workgroup quantizes it for its own weight type). */
static void qk_dec_group(qk_dec *D, const struct slm_tensor **ts, const void **devs, float **ys, int n,
                         const float *x, const void *xq) {
    int all_k = 1;
    for (int i = 0; i < n; i++) all_k &= ts[i]->type != GGUF_TT_Q8_0;
    if (all_k) {
        qk_gemv_desc d[QK_DEC_MAX_PROJ];
        for (int i = 0; i < n; i++) {
            d[i].type = ts[i]->type;
            d[i].pad_ = 0;
            d[i].n = ts[i]->shape[1];
            d[i].k = ts[i]->shape[0];
            d[i].w = devs[i];
            d[i].xq = xq;
            d[i].y = ys[i];
        }
        qk_dec_lib(hip_matvec_group(d, n, D->s), "grouped GEMV");
    } else {
        qk_gemv_desc_f32 d[QK_DEC_MAX_PROJ];
        for (int i = 0; i < n; i++) {
            d[i].type = ts[i]->type;
            d[i].pad_ = 0;
            d[i].n = ts[i]->shape[1];
            d[i].k = ts[i]->shape[0];
            d[i].w = devs[i];
            d[i].x = x;
            d[i].y = ys[i];
        }
        qk_dec_lib(hip_matvec_group_f32(d, n, D->s), "grouped GEMV (fp32 rows)");
    }
}

static void qk_dec_sync(qk_dec *D) {
    qk_dec_ck(hipStreamSynchronize(D->s), "hipStreamSynchronize");
    D->syncs++;
}

/* slm_forward_step for token tok at position pos, then the pick: with
 * sp NULL sample_argmax fused into the LM head, else sample_with
 * (hip_sample) on the device logits with the device rng and history, the
 * pick appended to the history. The logits as the forward pass left them
 * are copied into logits_host when it is not NULL. */
static int32_t qk_decode_step(struct slm_ctx *c, qk_dec *D, int32_t tok, int32_t pos, float *logits_host,
                              const struct slm_sampler *sp) {
    struct arena *a = c->arena;
    arena_reset(a);
    const struct slm_model *m = c->model;
    const int64_t H = D->hidden, F = D->ffn;
    hipStream_t s = D->s;
    const size_t row_bytes = (size_t)(H / QK_K) * 210;
    qk_dec_lib(hip_dequant_q6k((const uint8_t *)hip_qk_device_weight(m->W.tok_embd.data) + (size_t)tok * row_bytes,
                               H / QK_K, D->h, s),
               "embedding dequant");
    const float *delta = NULL;
    for (int32_t L = 0; L < m->cfg.n_layers; L++) {
        const struct slm_layer *Lw = &m->W.layers[L];
        /* h += ffn_out; x = attn_norm(h); the in-projections */
        qk_dec_lib(hip_add_rmsnorm_q8k(D->h, delta, D->attn_norm[L], D->eps, 1, H, D->h, D->xn, D->xq, s),
                   "attn_norm");
        const struct slm_tensor *ts[QK_DEC_MAX_PROJ];
        int n = 0;
        if (Lw->is_ssm) {
            ts[n++] = &Lw->attn_qkv;
            ts[n++] = &Lw->attn_gate;
            ts[n++] = &Lw->ssm_beta;
            ts[n++] = &Lw->ssm_alpha;
        } else {
            ts[n++] = &Lw->attn_q;
            ts[n++] = &Lw->attn_k;
            ts[n++] = &Lw->attn_v;
        }
        const void *devs[QK_DEC_MAX_PROJ];
        float *ys[QK_DEC_MAX_PROJ];
        for (int i = 0; i < n; i++) {
            devs[i] = qk_dec_weight(ts[i]);
            ys[i] = D->proj[i].y_dev;
        }
        qk_dec_group(D, ts, devs, ys, n, D->xn, D->xq);
        qk_dec_ck(hipMemcpyAsync(D->h_host, D->h, (size_t)H * 4, hipMemcpyDeviceToHost, s), "h to host");
        qk_dec_ck(hipMemcpyAsync(D->xn_host, D->xn, (size_t)H * 4, hipMemcpyDeviceToHost, s), "x to host");
        for (int i = 0; i < n; i++)
            qk_dec_ck(hipMemcpyAsync(D->proj[i].y_host, ys[i], (size_t)ts[i]->shape[1] * 4, hipMemcpyDeviceToHost, s),
                      "projection to host");
        qk_dec_sync(D);
        qk_seam_prefetch_clear();
        for (int i = 0; i < n; i++)
            qk_seam_prefetch_add(ts[i]->data, ts[i]->shape[1], ts[i]->shape[0], D->xn_host, D->proj[i].y_host);

        /* the reference's mixer on the host */
        struct tensor *h = tensor_new_2d(a, H, 1);
        memcpy(h->data, D->h_host, (size_t)H * 4);
        struct tensor *mix = Lw->is_ssm ? slm_forward_ssm(c, L, h) : slm_forward_attn(c, L, pos, h);
        qk_seam_prefetch_clear();

        /* FFN: h += mix; x = ffn_norm(h); down(silu(gate(x)) * up(x)) */
        memcpy(D->mix_host, mix->data, (size_t)H * 4);
        qk_dec_ck(hipMemcpyAsync(D->mix, D->mix_host, (size_t)H * 4, hipMemcpyHostToDevice, s), "mix to device");
        const struct slm_tensor *fg[2] = {&Lw->ffn_gate, &Lw->ffn_up};
        const void *fd[2] = {qk_dec_weight(fg[0]), qk_dec_weight(fg[1])};
        float *fy[2] = {D->gate, D->up};
        const int ffn_k = fg[0]->type != GGUF_TT_Q8_0 && fg[1]->type != GGUF_TT_Q8_0;
        qk_dec_lib(hip_add_rmsnorm_q8k(D->h, D->mix, D->ffn_norm[L], D->eps, 1, H, D->h, ffn_k ? NULL : D->xn,
                                       ffn_k ? D->xq : NULL, s),
                   "ffn_norm");
        qk_dec_group(D, fg, fd, fy, 2, D->xn, D->xq);
        const struct slm_tensor *dn[1] = {&Lw->ffn_down};
        const void *dd[1] = {qk_dec_weight(dn[0])};
        float *dy[1] = {D->ffn_out};
        const int down_k = dn[0]->type != GGUF_TT_Q8_0;
        qk_dec_lib(hip_swiglu_q8k(D->gate, D->up, 1, F, down_k ? NULL : D->act, down_k ? D->aq : NULL, s), "swiglu");
        qk_dec_group(D, dn, dd, dy, 1, D->act, D->aq);
        delta = D->ffn_out;
    }
    /* h += ffn_out; output_norm; LM head + greedy pick */
    qk_dec_lib(hip_add_rmsnorm_q8k(D->h, delta, D->out_norm, D->eps, 1, H, D->h, NULL, D->xq, s), "output_norm");
    const int sampled = sp != NULL;
    qk_dec_lib(hip_lmhead_q6k_argmax_topk(hip_qk_device_weight(m->W.output.data), D->vocab, H, D->xq, 0,
                                          (logits_host || sampled) ? D->logits : NULL, D->am, NULL, NULL, s),
               "LM head");
    if (logits_host)
        qk_dec_ck(hipMemcpyAsync(logits_host, D->logits, (size_t)D->vocab * 4, hipMemcpyDeviceToHost, s),
                  "logits to host");
    int32_t *pick = D->am;
    if (sampled) {
        if (D->hist_n >= D->hist_cap) {
            fprintf(stderr, "qk_decode: history full\n");
            abort();
        }
        qk_sampler q = {sp->temperature, sp->top_k, sp->top_p, sp->min_p, sp->repetition_penalty,
                        sp->repetition_window};
        pick = D->hist + D->hist_n;
        qk_dec_lib(hip_sample(D->logits, D->vocab, &q, D->rng, D->hist, D->hist_n, NULL, 0, pick, s), "sample");
        D->hist_n++;
    }
    qk_dec_ck(hipMemcpyAsync(D->am_host, pick, sizeof(int32_t), hipMemcpyDeviceToHost, s), "token to host");
    qk_dec_sync(D);
    return *D->am_host;
}
