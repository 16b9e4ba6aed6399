/*
 * ref_shim.c -- exports the reference's own quantized-matmul functions
 * from a shared library built out of the reference sources where they
 * lie (REF/slm/qwen.c and everything it includes; nothing is copied).
 *
 * TEST INFRASTRUCTURE ONLY: loaded by tests/ (to pin the C oracle) and
 * by bench.py's cpu_baseline leg (kind "reference"). Built by
 * oracle/Makefile with the reference's own flags (slm/Makefile:13-17:
 * clang -O3 -std=c17 -fvectorize -fslp-vectorize, no -march) into
 * oracle/_ref/libqkref.so.
 */
#include "qwen.c"
#include "sampler.c"   /* guarded by SAMPLER_C; topk_collect */

#include <pthread.h>

void ref_simd_init(void) { simd_init(); }
const char *ref_dispatch_label(void) { return simd_dispatch_label(); }

/* Which x86 tiers this CPU can run (bit t set = tier t usable;
 * 0 scalar, 1 AVX1, 2 AVX2-FMA, 3 AVX-VNNI), simd/simd.c:208-229. */
int ref_tiers_available(void) {
    simd_init();
    int m = 1;
#if defined(SIMD_X86)
    if (g_cpu.x86_avx) m |= 2;
    if (g_cpu.x86_avx2 && g_cpu.x86_fma) m |= 4;
    if (g_cpu.x86_avx_vnni && g_cpu.x86_avx2 && g_cpu.x86_fma) m |= 8;
#endif
    return m;
}

void ref_quantize_q8k(const float *x, void *y, int64_t k) {
    quantize_row_q8_K(x, (q8k_block *)y, k);
}
void ref_quantize_q8k_quants_h(const float *x, void *y, int64_t k) {
    q_quantize_row_q8_K(x, (q8k_block *)y, k);
}
void ref_quantize_q8_0(const float *x, void *y, int64_t k) {
    tensor_quantize_row_q8_0(x, (q8_0_block *)y, k);
}

/* tier -1: the dispatched entry point; 0..3: one tier by name. A tier
 * the CPU cannot run returns NaN instead of executing it. */
static int tier_ok(int tier) { return tier < 0 || ((ref_tiers_available() >> tier) & 1); }

float ref_q4k_dot(int tier, int nb, const void *w, const void *x) {
    const q4k_block *a = w; const q8k_block *b = x;
    float r = NAN;
    if (!tier_ok(tier)) return r;
    switch (tier) {
        case -1: r = simd_q4k_row_dot_q8k(nb, a, b); break;
        case 0:  r = q_scalar_q4k_row_dot_q8k(nb, a, b); break;
#if defined(SIMD_X86)
        case 1:  r = q4k_row_dot_q8k_avx1(nb, a, b); break;
        case 2:  r = q4k_row_dot_q8k_avx2(nb, a, b); break;
        case 3:  r = q4k_row_dot_q8k_avxvnni(nb, a, b); break;
#endif
        default: break;
    }
    return r;
}

float ref_q5k_dot(int tier, int nb, const void *w, const void *x) {
    const q5k_block *a = w; const q8k_block *b = x;
    float r = NAN;
    if (!tier_ok(tier)) return r;
    switch (tier) {
        case -1: r = simd_q5k_row_dot_q8k(nb, a, b); break;
        case 0:  r = q_scalar_q5k_row_dot_q8k(nb, a, b); break;
#if defined(SIMD_X86)
        case 1:  r = q5k_row_dot_q8k_avx1(nb, a, b); break;
        case 2:  r = q5k_row_dot_q8k_avx2(nb, a, b); break;
        case 3:  r = q5k_row_dot_q8k_avxvnni(nb, a, b); break;
#endif
        default: break;
    }
    return r;
}

float ref_q6k_dot(int tier, int nb, const void *w, const void *x) {
    const q6k_block *a = w; const q8k_block *b = x;
    float r = NAN;
    if (!tier_ok(tier)) return r;
    switch (tier) {
        case -1: r = simd_q6k_row_dot_q8k(nb, a, b); break;
        case 0:  r = q_scalar_q6k_row_dot_q8k(nb, a, b); break;
#if defined(SIMD_X86)
        case 1:  r = q6k_row_dot_q8k_avx1(nb, a, b); break;
        case 2:  r = q6k_row_dot_q8k_avx2(nb, a, b); break;
        case 3:  r = q6k_row_dot_q8k_avxvnni(nb, a, b); break;
#endif
        default: break;
    }
    return r;
}

float ref_q8_0_dot(int tier, int64_t k, const void *w, const void *x) {
    const q8_0_block *a = w; const q8_0_block *b = x;
    float r = NAN;
    if (!tier_ok(tier)) return r;
    switch (tier) {
        case -1: r = simd_q8_0_dot_q8_0(a, b, k); break;
        case 0:  r = q_scalar_q8_0_dot_q8_0(a, b, k); break;
#if defined(SIMD_X86)
        case 1:  r = q8_0_dot_q8_0_avx1(a, b, k); break;
        case 2:  r = q8_0_dot_q8_0_avx2(a, b, k); break;
        case 3:  r = q8_0_dot_q8_0_avxvnni(a, b, k); break;
#endif
        default: break;
    }
    return r;
}

void ref_dequant_q4k(const void *w, int64_t nb, float *y) {
    for (int64_t i = 0; i < nb; i++) q4k_dequant_block((const q4k_block *)w + i, y + i * QK_K);
}
void ref_dequant_q5k(const void *w, int64_t nb, float *y) {
    for (int64_t i = 0; i < nb; i++) q5k_dequant_block((const q5k_block *)w + i, y + i * QK_K);
}
void ref_dequant_q6k(const void *w, int64_t nb, float *y) {
    for (int64_t i = 0; i < nb; i++) q6k_dequant_block((const q6k_block *)w + i, y + i * QK_K);
}
void ref_scale_min(const uint8_t *s, int j, uint8_t *sc, uint8_t *m) {
    q4k_get_scale_min(s, j, sc, m);
}

/* tensor_matmul_*_f32 (slm/tensor.c:827-1033) called as the model
 * calls it through matmul_dispatch (slm/model.c:220-264): x is m rows
 * of k floats, out receives the (n, m) result tensor's data. */
int ref_matmul(int type, const void *w, int64_t n, int64_t k,
               const float *x, int64_t m, float *out) {
    simd_init();
    struct arena *a = arena_new((size_t)(m * k + m * n) * sizeof(float) + (1u << 20));
    struct tensor *xt = tensor_new_2d(a, k, m);
    memcpy(xt->data, x, (size_t)(m * k) * sizeof(float));
    struct tensor *r = NULL;
    switch (type) {
        case GGUF_TT_Q4_K: r = tensor_matmul_q4k_f32((const q4k_block *)w, n, k, xt); break;
        case GGUF_TT_Q5_K: r = tensor_matmul_q5k_f32((const q5k_block *)w, n, k, xt); break;
        case GGUF_TT_Q6_K: r = tensor_matmul_q6k_f32((const q6k_block *)w, n, k, xt); break;
        case GGUF_TT_Q8_0: r = tensor_matmul_q8_0_f32((const q8_0_block *)w, n, k, xt); break;
        default: break;
    }
    if (r) memcpy(out, r->data, (size_t)(m * n) * sizeof(float));
    arena_free(a);
    return r ? 0 : -1;
}

/* Harness-side row split for the N-core CPU baseline: quantize each
 * token once with the reference quantizer, then hand row ranges to
 * threads that call the unmodified dispatched simd_q*_row_dot. Rows
 * are independent (slm/tensor.c:846), so the output is bit-identical
 * to ref_matmul. */
struct rows_job {
    int type; const void *w; int64_t n, k, nb; const void *xq; float *out;
    int64_t r0, r1;
};

static void *rows_worker(void *p) {
    struct rows_job *j = p;
    for (int64_t r = j->r0; r < j->r1; r++) {
        float v = 0.0f;
        switch (j->type) {
            case GGUF_TT_Q4_K: v = simd_q4k_row_dot_q8k((int)j->nb, (const q4k_block *)j->w + r * j->nb, j->xq); break;
            case GGUF_TT_Q5_K: v = simd_q5k_row_dot_q8k((int)j->nb, (const q5k_block *)j->w + r * j->nb, j->xq); break;
            case GGUF_TT_Q6_K: v = simd_q6k_row_dot_q8k((int)j->nb, (const q6k_block *)j->w + r * j->nb, j->xq); break;
            default:           v = simd_q8_0_dot_q8_0((const q8_0_block *)j->w + r * j->nb, j->xq, j->k); break;
        }
        j->out[r] = v;
    }
    return NULL;
}

int ref_matmul_threads(int type, const void *w, int64_t n, int64_t k,
                       const float *x, int64_t m, float *out, int nthreads) {
    simd_init();
    if (nthreads < 1) nthreads = 1;
    if (nthreads > 256) nthreads = 256;
    int q8_0 = (type == GGUF_TT_Q8_0);
    int64_t nb = q8_0 ? k / QK8_0 : k / QK_K;
    size_t xbytes = q8_0 ? (size_t)nb * sizeof(q8_0_block) : (size_t)nb * sizeof(q8k_block);
    void *xq = malloc(xbytes);
    pthread_t th[256];
    struct rows_job jobs[256];
    if (!xq) return -1;
    for (int64_t t = 0; t < m; t++) {
        if (q8_0) tensor_quantize_row_q8_0(x + t * k, xq, k);
        else      quantize_row_q8_K(x + t * k, xq, k);
        for (int i = 0; i < nthreads; i++) {
            jobs[i] = (struct rows_job){type, w, n, k, nb, xq, out + t * n,
                                        n * i / nthreads, n * (i + 1) / nthreads};
            if (nthreads == 1) rows_worker(&jobs[i]);
            else pthread_create(&th[i], NULL, rows_worker, &jobs[i]);
        }
        if (nthreads > 1)
            for (int i = 0; i < nthreads; i++) pthread_join(th[i], NULL);
    }
    free(xq);
    return 0;
}

/* The same row split on a persistent pool: nthreads - 1 workers are
 * started once and spin (with pause) on a job generation counter, the
 * calling thread takes the first row range, so a call costs no thread
 * creation. Used by the N-core CPU baseline, where per-call thread
 * creation would cost more than a decode GEMV's rows. ref_pool_stop()
 * ends the workers. */
#include <sched.h>
#include <stdatomic.h>

static struct {
    int n;                                 /* workers (excluding the caller) */
    pthread_t th[256];
    struct rows_job jobs[256];
    atomic_uint gen;
    atomic_int done;
    atomic_int stop;
} g_pool;

static void *pool_worker(void *p) {
    const int id = (int)(intptr_t)p;
    unsigned seen = 0;
    for (;;) {
        unsigned g;
        int spins = 0;
        while ((g = atomic_load_explicit(&g_pool.gen, memory_order_acquire)) == seen) {
            if (atomic_load_explicit(&g_pool.stop, memory_order_relaxed)) return NULL;
            if (++spins < 4096) __builtin_ia32_pause();
            else sched_yield();
        }
        seen = g;
        rows_worker(&g_pool.jobs[id]);
        atomic_fetch_add_explicit(&g_pool.done, 1, memory_order_acq_rel);
    }
}

void ref_pool_stop(void) {
    if (g_pool.n == 0) return;
    atomic_store(&g_pool.stop, 1);
    for (int i = 1; i <= g_pool.n; i++) pthread_join(g_pool.th[i], NULL);
    g_pool.n = 0;
    atomic_store(&g_pool.stop, 0);
}

static int pool_start(int workers) {
    if (g_pool.n == workers) return 0;
    ref_pool_stop();
    atomic_store(&g_pool.gen, 0);
    for (int i = 1; i <= workers; i++) {
        if (pthread_create(&g_pool.th[i], NULL, pool_worker, (void *)(intptr_t)i) != 0) {
            g_pool.n = i - 1;
            ref_pool_stop();
            return -1;
        }
        g_pool.n = i;
    }
    return 0;
}

int ref_matmul_pool(int type, const void *w, int64_t n, int64_t k,
                    const float *x, int64_t m, float *out, int nthreads) {
    simd_init();
    if (nthreads < 1) nthreads = 1;
    if (nthreads > 256) nthreads = 256;
    if (pool_start(nthreads - 1) != 0) return -1;
    int q8_0 = (type == GGUF_TT_Q8_0);
    int64_t nb = q8_0 ? k / QK8_0 : k / QK_K;
    size_t xbytes = q8_0 ? (size_t)nb * sizeof(q8_0_block) : (size_t)nb * sizeof(q8k_block);
    void *xq = malloc(xbytes);
    if (!xq) return -1;
    for (int64_t t = 0; t < m; t++) {
        if (q8_0) tensor_quantize_row_q8_0(x + t * k, xq, k);
        else      quantize_row_q8_K(x + t * k, xq, k);
        for (int i = 0; i < nthreads; i++)
            g_pool.jobs[i] = (struct rows_job){type, w, n, k, nb, xq, out + t * n,
                                               n * i / nthreads, n * (i + 1) / nthreads};
        atomic_store_explicit(&g_pool.done, 0, memory_order_relaxed);
        atomic_fetch_add_explicit(&g_pool.gen, 1, memory_order_release);
        rows_worker(&g_pool.jobs[0]);
        while (atomic_load_explicit(&g_pool.done, memory_order_acquire) < nthreads - 1)
            __builtin_ia32_pause();
    }
    free(xq);
    return 0;
}

/* sample_argmax (slm/model.c:401) and topk_collect (slm/sampler.c:70)
 * on a 1-D view of v. */
static struct tensor view1d(const float *v, int64_t n) {
    struct tensor t;
    memset(&t, 0, sizeof(t));
    t.ndim = 1;
    t.ne[0] = n;
    for (int i = 1; i < TENSOR_MAX_DIMS; i++) t.ne[i] = 1;
    t.nb[0] = sizeof(float);
    t.data = (float *)v;
    return t;
}

int32_t ref_argmax(const float *v, int64_t n) {
    struct tensor t = view1d(v, n);
    return sample_argmax(&t);
}

int32_t ref_topk_collect(const float *v, int64_t n, int32_t k, int32_t *idx, float *val) {
    struct tensor t = view1d(v, n);
    return topk_collect(&t, k, idx, val);
}

/* tensor_add then tensor_rms_norm (slm/tensor.c:284, 345) on m rows of k
 * floats, through the reference's arena; delta may be NULL. */
int ref_add_rmsnorm(const float *h, const float *delta, const float *w, float eps,
                    int64_t m, int64_t k, float *h_out, float *x_out) {
    struct arena *a = arena_new((size_t)(4 * m * k + 4 * k) * sizeof(float) + (1u << 16));
    if (!a) return -1;
    struct tensor *x = tensor_new_2d(a, k, m);
    memcpy(x->data, h, (size_t)(m * k) * sizeof(float));
    if (delta) {
        struct tensor *d = tensor_new_2d(a, k, m);
        memcpy(d->data, delta, (size_t)(m * k) * sizeof(float));
        x = tensor_add(x, d);
    }
    struct tensor *wt = tensor_new_1d(a, k);
    memcpy(wt->data, w, (size_t)k * sizeof(float));
    struct tensor *y = tensor_rms_norm(x, wt, eps);
    memcpy(h_out, x->data, (size_t)(m * k) * sizeof(float));
    memcpy(x_out, y->data, (size_t)(m * k) * sizeof(float));
    arena_free(a);
    return 0;
}

/* simd_silu_f32 (simd/simd.c:271) and tensor_mul (slm/tensor.c:293). */
void ref_silu(int64_t n, const float *x, float *y) { simd_silu_f32((int)n, y, x); }

int ref_swiglu(int64_t n, const float *gate, const float *up, float *act) {
    struct arena *a = arena_new((size_t)(3 * n) * sizeof(float) + (1u << 16));
    if (!a) return -1;
    struct tensor *g = tensor_new_1d(a, n), *u = tensor_new_1d(a, n);
    memcpy(u->data, up, (size_t)n * sizeof(float));
    simd_silu_f32((int)n, g->data, gate);
    struct tensor *o = tensor_mul(g, u);
    memcpy(act, o->data, (size_t)n * sizeof(float));
    arena_free(a);
    return 0;
}

/* sample_with (slm/sampler.c:134) on a 1-D view of logits (modified in
 * place, as the reference does), between the min_new masking of
 * slm_generate_raw and its restore of the masked values
 * (slm/slm.c:309-333); st holds struct rng's two words and is advanced.
 * rng_seed (slm/model.c:431) for the tests' seeds. */
int32_t ref_sample(float *logits, int64_t n, float temperature, int32_t top_k, float top_p, float min_p,
                   float penalty, int32_t window, uint64_t *st, const int32_t *history, int32_t hist_n,
                   const int32_t *mask, int32_t n_mask) {
    struct tensor t = view1d(logits, n);
    struct slm_sampler sp;
    sp.temperature = temperature;
    sp.top_k = top_k;
    sp.top_p = top_p;
    sp.min_p = min_p;
    sp.repetition_penalty = penalty;
    sp.repetition_window = window;
    float saved[n_mask > 0 ? n_mask : 1];
    for (int32_t i = 0; i < n_mask; i++)
        if (mask[i] >= 0 && mask[i] < n) {
            saved[i] = logits[mask[i]];
            logits[mask[i]] = -INFINITY;
        }
    struct rng r;
    r.s0 = st[0];
    r.s1 = st[1];
    int32_t tok = sample_with(&t, &sp, &r, history, hist_n);
    st[0] = r.s0;
    st[1] = r.s1;
    for (int32_t i = 0; i < n_mask; i++)
        if (mask[i] >= 0 && mask[i] < n) logits[mask[i]] = saved[i];
    return tok;
}

void ref_rng_seed(uint64_t seed, uint64_t *st) {
    struct rng r;
    rng_seed(&r, seed);
    st[0] = r.s0;
    st[1] = r.s1;
}

/* chunked_ssm_step_f32 (slm/chunked.c:287) with scratch of its own. */
void ref_chunked_step(int n, int kd, int vd, const float *q, const float *k, const float *v, const float *g,
                      const float *beta, float *state, float *out) {
    const size_t C = CHUNK_SIZE, NK = C * (size_t)kd, NV = C * (size_t)vd, CC = C * C;
    float *buf = (float *)calloc(2 * C + 6 * CC + 6 * NK + 8 * NV + (size_t)kd * vd, sizeof(float));
    float *p = buf;
    float *gcs = p; p += C;
    float *gexp = p; p += C;
    float *dm = p; p += CC;
    float *kb = p; p += NK;
    float *vb = p; p += NV;
    float *kkd = p; p += CC;
    float *lhs = p; p += CC;
    float *attn = p; p += CC;
    float *veff = p; p += NV > CC ? NV : CC;
    float *kbg = p; p += NK;
    float *kcd = p; p += NK;
    float *akq = p; p += CC;
    float *qg = p; p += NK;
    float *ai = p; p += NV;
    float *vp = p; p += NV;
    float *vn = p; p += NV;
    float *va = p; p += NV;
    float *kgd = p; p += NK;
    float *kv = p;
    chunked_ssm_step_f32(n, kd, vd, q, k, v, g, beta, state, out, gcs, gexp, dm, kb, vb, kkd, lhs, attn, veff,
                         kbg, kcd, akq, qg, ai, vp, vn, va, kgd, kv);
    free(buf);
}
