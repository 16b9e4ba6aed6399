/*
 * qk_oracle.h -- CPU restatement of qwen.haiku's quantized matmul path.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the checker for libqk: only
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load it. Nothing in the product path (include/qk.h, qwen.haiku_amd/)
 * links or calls it.
 *
 * Plain C99, built with gcc at -O2 -ffp-contract=off: every float op
 * rounds separately unless the function calls fmaf() explicitly, which
 * is where the reference's AVX2/AVX-VNNI tier contracts to an FMA.
 * Block layouts are the ones in include/qk.h (simd/quants.h:95-130).
 */
#ifndef QK_ORACLE_H
#define QK_ORACLE_H

#include <stdint.h>

/* Epilogue families: 0 = scalar / AVX1 (separately rounded ops),
 * 1 = AVX2-FMA / AVX-VNNI (fused Q4_K/Q5_K term, 8-lane Q8_0). */
#define QKO_EPI_SEPARATE 0
#define QKO_EPI_FUSED    1

float    qko_f16_to_f32(uint16_t h);
uint16_t qko_f32_to_f16(float f);
int32_t  qko_nearest_int(float v);

void qko_quantize_q8k(const float *x, void *xq, int64_t k);
void qko_quantize_q8_0(const float *x, void *xq, int64_t k);
void qko_scale_min(const uint8_t *s, int j, uint8_t *sc, uint8_t *m);

float qko_q4k_dot(int nb, const void *w, const void *xq, int epi);
float qko_q5k_dot(int nb, const void *w, const void *xq, int epi);
float qko_q6k_dot(int nb, const void *w, const void *xq, int epi);
float qko_q8_0_dot(int64_t k, const void *w, const void *xq, int epi);

/* Integer parts of one super-block dot (no float epilogue). */
void qko_q4k_block_ints(const void *w, const void *xq, int32_t *isum,
                        int32_t *isum_mins);
void qko_q5k_block_ints(const void *w, const void *xq, int32_t *isum,
                        int32_t *isum_mins);
void qko_q6k_block_ints(const void *w, const void *xq, int32_t *isum,
                        int32_t *isum_mins);

void qko_dequant_q4k(const void *w, int64_t nblocks, float *y);
void qko_dequant_q5k(const void *w, int64_t nblocks, float *y);
void qko_dequant_q6k(const void *w, int64_t nblocks, float *y);

/* out[t*n + j] for t < m, j < n; type is a GGUF id (8, 12, 13, 14).
 * Rows [row0, row1) only, so callers can split rows across threads. */
int qko_matmul(int type, const void *w, int64_t n, int64_t k,
               const float *x, int64_t m, float *out, int epi,
               int64_t row0, int64_t row1);
/* Same with pre-quantized activations (m rows of Q8_K / Q8_0). */
int qko_matmul_xq(int type, const void *w, int64_t n, int64_t k,
                  const void *xq, int64_t m, float *out, int epi,
                  int64_t row0, int64_t row1);

/* Decode-chain links: residual add + RMSNorm (h_out gets h + delta,
 * x_out the normalized rows; delta may be NULL), SiLU, SiLU(gate)*up. */
void qko_add_rmsnorm(const float *h, const float *delta, const float *w,
                     float eps, int64_t m, int64_t k, float *h_out,
                     float *x_out);
void qko_silu(int64_t n, const float *x, float *y);
void qko_swiglu(int64_t n, const float *gate, const float *up, float *act);

int32_t qko_argmax(const float *v, int64_t n);

/* Chunked Gated DeltaNet: one chunk of one head (n <= 64, kd, vd <= 128),
 * and the chunk loop over all heads of a layer. */
void qko_chunked_step(int n, int kd, int vd, const float *q, const float *k, const float *v, const float *g,
                      const float *beta, float *state, float *out);
void qko_deltanet_chunked(int64_t n_tok, int n_heads, int kd, int vd, const float *q, const float *k,
                          const float *v, const float *g, const float *beta, float *state, float *out);

/* Sampler chain (sample_with plus the min_new masking); st is the
 * reference's two-word rng state, advanced on the sampling path. */
void qko_rng_seed(uint64_t seed, uint64_t *st);
int32_t qko_sample(float *logits, int64_t n, float temperature, int32_t top_k, float top_p, float min_p,
                   float penalty, int32_t window, uint64_t *st, const int32_t *history, int32_t hist_n,
                   const int32_t *mask, int32_t n_mask);
int32_t qko_topk_collect(const float *v, int64_t n, int32_t k,
                         int32_t *idx, float *val);

#endif
