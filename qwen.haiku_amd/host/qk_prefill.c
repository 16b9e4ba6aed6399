/*
 * qk_prefill.c -- the batched prefill of the hybrid Qwen3.5 forward pass
 * with each Gated DeltaNet layer's chunk loop in one GPU call.
 *
 * Included by qwen_e2e.c in its GPU build, after the reference's qwen.c
 * and after qk_seam.c. It is the change a maintainer makes next to the
 * seam: through the seam alone, slm_forward_ssm_batch (slm/qwen.c:627-855)
 * hands the GPU one head of one 64-token chunk per call
 * (chunked_ssm_step_f32, slm/chunked.c:287), n_heads x n/64 host round
 * trips per layer (2304 for a 512-token prompt on the 0.8B shape). The
 * loop's operands are already laid out the way hip_deltanet_chunked
 * takes them (Q/K (n, heads, k_hd), V and the output (n, heads, v_hd),
 * beta and the log-gates (n, heads), the layer's state (heads, k_hd,
 * v_hd)), so qk_ssm_batch below runs the whole loop, every chunk of every
 * head with the state carried, as one hip_qk_deltanet_layer_host call.
 *
 * Everything else is the reference's arithmetic in the reference's order
 * (slm/qwen.c:627-720 and 815-855 for the SSM layer, 1018-1103 for the
 * pass), calling the reference's own helpers (tensor_rms_norm,
 * matmul_dispatch, which reaches the seam, simd_silu_f32, tensor_add,
 * tensor_mul, the attention mixer slm_forward_attn_batch), so the
 * logits and the state are the reference's bit for bit and the token
 * stream is unchanged.
 */

/* Seconds inside the per-layer DeltaNet calls (added to the seam's count). */
static double qk_prefill_layer_calls;

/* slm_forward_ssm_batch with the chunk loop (its step 9) in one call. */
static struct tensor *qk_ssm_batch(struct slm_ctx *c, int32_t L, int32_t n, struct tensor *h) {
    struct arena *a = c->arena;
    const struct slm_config *cf = &c->model->cfg;
    struct slm_layer *Lw = &c->model->W.layers[L];
    const int32_t H = cf->linear_n_heads, kd = cf->linear_k_head_dim, vd = cf->linear_v_head_dim;
    const int32_t kdim = H * kd, vdim = H * vd, taps = cf->linear_conv_kernel;
    const int32_t cdim = 2 * kdim + vdim;
    assert(n > 0);
    /* norm and in-projections (slm/qwen.c:639-650) */
    struct tensor nw = weights_as_f32_view(&Lw->attn_norm, a);
    struct tensor *xn = tensor_rms_norm(h, &nw, cf->norm_eps);
    struct tensor *qkv = matmul_dispatch(&Lw->attn_qkv, xn);
    struct tensor *z = matmul_dispatch(&Lw->attn_gate, xn);
    struct tensor *bt = matmul_dispatch(&Lw->ssm_beta, xn);
    struct tensor *at = matmul_dispatch(&Lw->ssm_alpha, xn);
    /* causal conv1d over the ring of the last `taps` rows, token by
       token (:658-678) */
    struct tensor *mixed = tensor_new_2d(a, cdim, n);
    const float *cw = (const float *)Lw->ssm_conv1d.data;
    float *ring = c->ssm.conv_state + (size_t)L * taps * cdim;
    for (int32_t t = 0; t < n; t++) {
        memcpy(ring + (size_t)c->ssm.conv_head[L] * cdim, qkv->data + (size_t)t * cdim,
               (size_t)cdim * sizeof(float));
        c->ssm.conv_head[L] = (c->ssm.conv_head[L] + 1) % taps;
        const int32_t oldest = c->ssm.conv_head[L];
        for (int32_t ch = 0; ch < cdim; ch++) {
            float acc = 0.0f;
            for (int32_t j = 0; j < taps; j++) acc += ring[(size_t)((oldest + j) % taps) * cdim + ch] * cw[(size_t)ch * taps + j];
            mixed->data[(size_t)t * cdim + ch] = acc;
        }
    }
    simd_silu_f32(n * cdim, mixed->data, mixed->data);
    /* split into Q, K, V rows; per head, Q and K scaled by their inverse
       L2 norms (Q also by 1/sqrt(k_hd)) (:684-717) */
    float *Q = ARENA_F32((size_t)n * kdim), *K = ARENA_F32((size_t)n * kdim), *V = ARENA_F32((size_t)n * vdim);
    for (int32_t t = 0; t < n; t++) {
        const float *row = mixed->data + (size_t)t * cdim;
        memcpy(Q + (size_t)t * kdim, row, (size_t)kdim * sizeof(float));
        memcpy(K + (size_t)t * kdim, row + kdim, (size_t)kdim * sizeof(float));
        memcpy(V + (size_t)t * vdim, row + 2 * kdim, (size_t)vdim * sizeof(float));
    }
    const float scale = 1.0f / sqrtf((float)kd);
    for (int32_t t = 0; t < n; t++) {
        for (int32_t hh = 0; hh < H; hh++) {
            float *q = Q + (size_t)t * kdim + (size_t)hh * kd, *k = K + (size_t)t * kdim + (size_t)hh * kd;
            double qs = 0.0, ks = 0.0;
            for (int32_t i = 0; i < kd; i++) {
                qs += (double)(q[i] * q[i]);
                ks += (double)(k[i] * k[i]);
            }
            const float qr = 1.0f / fmaxf(sqrtf((float)qs), 1e-6f), kr = 1.0f / fmaxf(sqrtf((float)ks), 1e-6f);
            for (int32_t i = 0; i < kd; i++) {
                q[i] *= qr * scale;
                k[i] *= kr;
            }
        }
    }
    /* beta = sigmoid(b), log-gate = a_log * softplus(alpha + dt_bias)
       (:721-733) */
    const float *alog = (const float *)Lw->ssm_a.data, *dtb = (const float *)Lw->ssm_dt_bias.data;
    float *beta = ARENA_F32((size_t)n * H), *glog = ARENA_F32((size_t)n * H);
    for (int32_t t = 0; t < n; t++) {
        for (int32_t hh = 0; hh < H; hh++) {
            const size_t i = (size_t)t * H + hh;
            beta[i] = 1.0f / (1.0f + expf(-bt->data[i]));
            const float x = at->data[i] + dtb[hh];
            glog[i] = alog[hh] * (x > 20.0f ? x : logf(1.0f + expf(x)));
        }
    }
    /* the chunk loop of every head, the layer's state carried in place
       (:773-812): one call */
    float *state = c->ssm.ssm_state + (size_t)L * H * kd * vd;
    float *out = ARENA_F32((size_t)n * vdim);
    const double t0 = qk_seam_now();
    const int rc = hip_qk_deltanet_layer_host(n, H, kd, vd, Q, K, V, glog, beta, state, out);
    qk_prefill_layer_calls += qk_seam_now() - t0;
    if (rc) {
        fprintf(stderr, "qk_prefill: hip_qk_deltanet_layer_host failed (%d): %s\n", rc, hip_qk_last_error());
        abort();
    }
    /* gated RMSNorm with SiLU(z) per head, then the out-projection
       (:815-853) */
    const float *sw = (const float *)Lw->ssm_norm.data;
    struct tensor *y = tensor_new_2d(a, vdim, n);
    float *zs = ARENA_F32((size_t)vdim);
    for (int32_t t = 0; t < n; t++) {
        simd_silu_f32(vdim, zs, z->data + (size_t)t * vdim);
        for (int32_t hh = 0; hh < H; hh++) {
            const float *o = out + (size_t)t * vdim + (size_t)hh * vd;
            float *yo = y->data + (size_t)t * vdim + (size_t)hh * vd;
            double ss = 0.0;
            for (int32_t v = 0; v < vd; v++) ss += (double)(o[v] * o[v]);
            const float rs = 1.0f / sqrtf((float)(ss / (double)vd) + cf->norm_eps);
            for (int32_t v = 0; v < vd; v++) yo[v] = o[v] * rs;
            for (int32_t v = 0; v < vd; v++) yo[v] = yo[v] * sw[v];
            for (int32_t v = 0; v < vd; v++) yo[v] = yo[v] * zs[(size_t)hh * vd + v];
        }
    }
    return matmul_dispatch(&Lw->ssm_out, y);
}

/* slm_forward_batch (slm/qwen.c:1018-1103) with qk_ssm_batch for the
 * SSM layers: embedding rows, per layer mixer + residual + SwiGLU FFN +
 * residual, then the final norm and the LM head on the last token. */
static struct tensor *qk_forward_batch(struct slm_ctx *c, const int32_t *ids, int32_t n, int32_t pos0) {
    assert(n > 0);
    struct arena *a = c->arena;
    arena_reset(a);
    const struct slm_config *cf = &c->model->cfg;
    const int32_t hd = cf->hidden_dim;
    struct tensor *h = tensor_new_2d(a, hd, n);
    for (int32_t t = 0; t < n; t++) {
        float *dst = h->data + (size_t)t * hd;
        if (c->model->W.tok_embd.type == GGUF_TT_F32) {
            memcpy(dst, (const float *)c->model->W.tok_embd.data + (size_t)ids[t] * hd, (size_t)hd * sizeof(float));
        } else {
            const int32_t nb = hd / QK_K;
            const q6k_block *row = (const q6k_block *)c->model->W.tok_embd.data + (size_t)ids[t] * nb;
            for (int32_t b = 0; b < nb; b++) q6k_dequant_block(row + b, dst + b * QK_K);
        }
    }
    for (int32_t L = 0; L < cf->n_layers; L++) {
        struct slm_layer *Lw = &c->model->W.layers[L];
        struct tensor *mix = Lw->is_ssm ? qk_ssm_batch(c, L, n, h) : slm_forward_attn_batch(c, L, pos0, n, h);
        h = tensor_add(h, mix);
        struct tensor fw = weights_as_f32_view(&Lw->ffn_norm, a);
        struct tensor *xn = tensor_rms_norm(h, &fw, cf->norm_eps);
        struct tensor *gate = matmul_dispatch(&Lw->ffn_gate, xn);
        struct tensor *up = matmul_dispatch(&Lw->ffn_up, xn);
        struct tensor *act = tensor_new_2d(a, gate->ne[0], gate->ne[1]);
        simd_silu_f32((int)tensor_nelements(gate), act->data, gate->data);
        h = tensor_add(h, matmul_dispatch(&Lw->ffn_down, tensor_mul(act, up)));
    }
    struct tensor *last = tensor_new_2d(a, hd, 1);
    memcpy(last->data, h->data + (size_t)(n - 1) * hd, (size_t)hd * sizeof(float));
    struct tensor ow = weights_as_f32_view(&c->model->W.output_norm, a);
    return matmul_dispatch(&c->model->W.output, tensor_rms_norm(last, &ow, cf->norm_eps));
}
