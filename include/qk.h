/*
 * qk.h -- C ABI of libqk, the MI355X (gfx950) quantized matmul path.
 *
 * libqk replaces the CPU SIMD dispatch behind qwen.haiku's quantized
 * tensor ops: GGUF Q4_K / Q5_K / Q6_K / Q8_0 weight rows multiplied
 * against activations quantized to Q8_K (Q8_0 for Q8_0 weights).
 * Every entry point is `extern "C"`, takes plain pointers and sizes, and
 * returns an int status (QK_OK == 0). On failure hip_qk_last_error()
 * returns a message for the calling thread.
 *
 * Two layers:
 *
 *  1. Device layer (hip_quantize_*, hip_matvec_*, hip_matmul_*,
 *     hip_dequant_*, hip_lmhead_*): every pointer is a device pointer;
 *     work is enqueued on `stream` (a hipStream_t, NULL = the null
 *     stream) and the call returns without synchronizing.
 *  2. Host seam (hip_qk_register_weight, hip_qk_matmul_host,
 *     hip_qk_lmhead_host): host pointers, synchronous. This is the body
 *     of the reference's tensor_matmul_*_f32 (slm/tensor.c:827-1033)
 *     moved onto the GPU; weights are uploaded once and found again by
 *     their host address, so the reference's call signatures need no
 *     change (qwen.haiku_amd/host/qk_seam.c).
 *
 * Results are bit-identical to the reference CPU path of the selected
 * tier (hip_qk_set_tier): the integer part of every row dot is exact,
 * and the float epilogue reproduces the rounding sequence of that tier.
 */
#ifndef QK_H
#define QK_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* libqk is built with hidden visibility; the entry points declared here
 * are the only names it exports into the host process. */
#pragma GCC visibility push(default)

/* Super-block / block sizes, simd/quants.h:30-31. */
#define QK_K  256
#define QK8_0 32

/* GGUF tensor type ids, slm/gguf.c:52-59. */
enum {
    QK_TYPE_F32  = 0,
    QK_TYPE_Q8_0 = 8,
    QK_TYPE_Q4_K = 12,
    QK_TYPE_Q5_K = 13,
    QK_TYPE_Q6_K = 14
};

/* Block layouts, byte-identical to simd/quants.h:95-130. fp16 fields are
 * carried as raw IEEE binary16 bits. */
typedef struct {
    float   d;                 /* 1 / iscale                        */
    int8_t  qs[QK_K];          /* 256 quants                        */
    int16_t bsums[QK_K / 16];  /* sums of 16-element groups         */
} qk_q8k_block;                /* 292 B                             */

typedef struct {
    uint16_t d, dmin;          /* fp16                              */
    uint8_t  scales[12];       /* 8 x (6-bit scale, 6-bit min)      */
    uint8_t  qs[QK_K / 2];     /* 4-bit quants                      */
} qk_q4k_block;                /* 144 B                             */

typedef struct {
    uint16_t d, dmin;
    uint8_t  scales[12];
    uint8_t  qh[QK_K / 8];     /* 5th bit                           */
    uint8_t  qs[QK_K / 2];
} qk_q5k_block;                /* 176 B                             */

typedef struct {
    uint8_t  ql[QK_K / 2];     /* low 4 bits                        */
    uint8_t  qh[QK_K / 4];     /* high 2 bits                       */
    int8_t   scales[QK_K / 16];
    uint16_t d;                /* fp16                              */
} qk_q6k_block;                /* 210 B                             */

typedef struct {
    uint16_t d;                /* fp16                              */
    int8_t   qs[QK8_0];
} qk_q8_0_block;               /* 34 B                              */

/* Status codes. */
enum {
    QK_OK               = 0,
    QK_ERR_ARG          = 1,   /* bad shape, null pointer, k % block   */
    QK_ERR_HIP          = 2,   /* a HIP runtime call failed            */
    QK_ERR_NOT_INIT     = 3,   /* hip_qk_init not called / failed      */
    QK_ERR_UNREGISTERED = 4,   /* host weight pointer not registered   */
    QK_ERR_NOMEM        = 5,
    QK_ERR_UNSUPPORTED  = 6    /* tensor type not on this path, or the */
                               /* host libm expf is not the FMA build  */
};

/* CPU dispatch tiers whose float epilogue the kernels reproduce
 * (simd/simd.c:208-229). SCALAR and AVX1 round every product and
 * difference separately; AVX2 and AVX-VNNI fuse d*isum - dmin*mins into
 * one FMA (Q4_K/Q5_K) and reduce Q8_0 over 8 FMA lanes. */
enum {
    QK_TIER_AUTO    = -1,      /* pick the tier this host CPU runs     */
    QK_TIER_SCALAR  = 0,
    QK_TIER_AVX1    = 1,
    QK_TIER_AVX2    = 2,
    QK_TIER_AVXVNNI = 3
};

/* ---- lifecycle ------------------------------------------------------ */

/* Select `device` and pick the tier (QK_TIER_AUTO). Replaces simd_init()
 * (simd/simd.c:191), called from slm_model_load (slm/model.c:1134).
 * Idempotent for the same device; another device needs hip_qk_shutdown
 * first. */
int         hip_qk_init(int device);
/* Wait for the device, then free every registered weight, every host
 * thread's seam stream and staging, and all scratch. */
void        hip_qk_shutdown(void);
/* "gfx950 <name> / tier AVX2-FMA"; replaces simd_dispatch_label()
 * (simd/simd.c:234). */
const char *hip_qk_device_label(void);
/* Message of the last failed call on this thread ("" if none). */
const char *hip_qk_last_error(void);
/* Force a tier (QK_TIER_*); QK_TIER_AUTO re-detects from CPUID the way
 * detect_cpu() does (simd/simd.c:142-170). */
int         hip_qk_set_tier(int tier);
int         hip_qk_get_tier(void);
/* Tier name as the reference labels it: "scalar", "AVX1", "AVX2-FMA",
 * "AVX-VNNI". */
const char *hip_qk_tier_label(int tier);

/* ---- device layer: activation quantizers --------------------------- */

/* m rows of k floats -> m * k/256 Q8_K blocks (row t at xq + t*k/256).
 * Bit-exact quantize_row_q8_K (slm/tensor.c:683-720). k % 256 == 0;
 * m * k/256 at most 2^26 blocks. */
int hip_quantize_q8k(const float *x, int64_t m, int64_t k, void *xq,
                     void *stream);
/* m rows of k floats -> m * k/32 Q8_0 blocks. Bit-exact
 * tensor_quantize_row_q8_0 (slm/tensor.c:930-950; roundf, half away
 * from zero). k % 32 == 0; m * k/32 at most 2^27 blocks. */
int hip_quantize_q8_0(const float *x, int64_t m, int64_t k, void *xq,
                      void *stream);

/* ---- device layer: decode GEMV (one activation row) ----------------- */

/* y[j] = row_dot(W row j, xq) for j < n. W is n rows of k/256 blocks in
 * native GGUF layout; xq is k/256 Q8_K blocks (k/32 Q8_0 blocks for
 * hip_matvec_q8_0). Replaces the LLM_PAR_FOR row loop of
 * tensor_matmul_q{4k,5k,6k}_f32 / _q8_0_f32 at n_tok == 1
 * (slm/tensor.c:846-850, 912-917, 1026-1031, 974-979) and the
 * simd_q*_row_dot entry points it calls (simd/simd.c:236-250).
 * Limits: w 16-byte aligned; k <= QK_MAX_K (a Q8_0 activation row is
 * staged in LDS; the limit holds for every type and every matvec /
 * matmul entry point); the matrix (n rows x row bytes) below 4 GB
 * (32-bit offsets). */
#define QK_MAX_K 65536
int hip_matvec_q4k (const void *w, int64_t n, int64_t k, const void *xq,
                    float *y, void *stream);
int hip_matvec_q5k (const void *w, int64_t n, int64_t k, const void *xq,
                    float *y, void *stream);
int hip_matvec_q6k (const void *w, int64_t n, int64_t k, const void *xq,
                    float *y, void *stream);
int hip_matvec_q8_0(const void *w, int64_t n, int64_t k, const void *xq,
                    float *y, void *stream);

/* One launch over several GEMVs (a decode layer's projections): entry i
 * computes y_i = W_i . xq_i as hip_matvec_<type_i> would. Descriptors
 * live in host memory and are copied into the launch's kernel
 * arguments; at most QK_GROUP_MAX entries. */
#define QK_GROUP_MAX 16
typedef struct {
    int32_t     type;          /* QK_TYPE_Q4_K / Q5_K / Q6_K / Q8_0   */
    int32_t     pad_;
    int64_t     n, k;
    const void *w;             /* device                              */
    const void *xq;            /* device                              */
    float      *y;             /* device                              */
} qk_gemv_desc;
int hip_matvec_group(const qk_gemv_desc *desc, int count, void *stream);

/* The same launch from fp32 activation rows: entry i computes
 * y_i = W_i . quant(x_i), x_i being k_i floats (16-byte aligned; 4-byte
 * for Q8_0). Each workgroup quantizes the row it needs into LDS, bit for
 * bit as hip_quantize_q8k / hip_quantize_q8_0 would, so a decode layer's
 * projections are one dispatch from the fp32 activations: the
 * quantize-then-dot of tensor_matmul_*_f32 at n_tok == 1
 * (slm/tensor.c:838-850) for up to QK_GROUP_MAX weights at once. Entries
 * may share an x. */
typedef struct {
    int32_t     type;
    int32_t     pad_;
    int64_t     n, k;
    const void *w;             /* device                              */
    const float *x;            /* device, k floats                    */
    float      *y;             /* device                              */
} qk_gemv_desc_f32;
int hip_matvec_group_f32(const qk_gemv_desc_f32 *desc, int count, void *stream);

/* ---- device layer: chunked-prefill GEMM ----------------------------- */

/* y[t*n + j] = row_dot(W row j, xq row t) for t < m, j < n: the token
 * loop of tensor_matmul_q{4k,5k,6k}_f32 (slm/tensor.c:838-851) as one
 * int8-MFMA GEMM. xq holds m rows of k/256 Q8_K blocks (k/32 Q8_0 blocks
 * for hip_matmul_q8_0, the token loop of tensor_matmul_q8_0_f32,
 * slm/tensor.c:952-981). m is at most 65535 * 64 (65535 * 32 for
 * hip_matmul_q8_0); so is n_tok of hip_qk_matmul_host. */
int hip_matmul_q4k(const void *w, int64_t n, int64_t k, const void *xq,
                   int64_t m, float *y, void *stream);
int hip_matmul_q5k(const void *w, int64_t n, int64_t k, const void *xq,
                   int64_t m, float *y, void *stream);
int hip_matmul_q6k(const void *w, int64_t n, int64_t k, const void *xq,
                   int64_t m, float *y, void *stream);
int hip_matmul_q8_0(const void *w, int64_t n, int64_t k, const void *xq,
                    int64_t m, float *y, void *stream);

/* ---- device layer: prefill GEMM over repacked weights --------------- */

/* No counterpart in the reference, whose weights stay in GGUF blocks; for
 * callers that run many prefill GEMMs on one weight matrix. Weights are
 * immutable after load (slm/slm.h:12-13), so a Q4_K / Q5_K / Q6_K matrix
 * can be repacked once into int8 MFMA planes (552 / 552 / 520 bytes per
 * row and super-block, against 144 / 176 / 210 for the blocks; the host
 * seam does this for every matrix it runs a prefill GEMM on).
 * hip_matmul_planes then computes exactly what hip_matmul_q4k / _q5k /
 * _q6k compute on the original blocks, bit for bit, without re-deriving
 * the operands for every token tile.
 * hip_gemm_planes_bytes: bytes of the planes of an n x k matrix, 0 for a
 * type or shape without planes. hip_gemm_pack_planes: w (device, native
 * blocks, 16-byte aligned) -> planes (device, that many bytes, 16-byte
 * aligned, not overlapping w). */
size_t hip_gemm_planes_bytes(int type, int64_t n, int64_t k);
int hip_gemm_pack_planes(int type, const void *w, int64_t n, int64_t k,
                         void *planes, void *stream);
int hip_matmul_planes(int type, const void *planes, int64_t n, int64_t k,
                      const void *xq, int64_t m, float *y, void *stream);

/* ---- device layer: dequantization ----------------------------------- */

/* nblocks blocks -> nblocks*256 floats. Bit-exact q{4,5,6}k_dequant_block
 * (slm/tensor.c:800-820, 867-896, 988-1010). nblocks at most 2^26. */
int hip_dequant_q4k(const void *w, int64_t nblocks, float *y, void *stream);
int hip_dequant_q5k(const void *w, int64_t nblocks, float *y, void *stream);
int hip_dequant_q6k(const void *w, int64_t nblocks, float *y, void *stream);

/* ---- device layer: the decode chain's elementwise links ------------- */

/* Residual add + RMSNorm (+ Q8_K), per row t < m of k floats:
 *   r = h + delta                 tensor_add, slm/tensor.c:284-291
 *                                 (delta may be NULL: r = h)
 *   x = rms_norm(r) * w           tensor_rms_norm, slm/tensor.c:345-367:
 *                                 the sequential double sum of (r_i*r_i),
 *                                 rscale = 1/sqrtf((float)(ssq/k) + eps),
 *                                 x_i = (r_i*rscale)*w_i
 *   xq = quantize_row_q8_K(x)     slm/tensor.c:683-720
 * h_out (may be NULL, may equal h) receives r, x_out (may be NULL) x,
 * xq (may be NULL, needs k % 256 == 0) the Q8_K row for the next GEMV;
 * one of x_out / xq is required. w holds k floats shared by every row.
 * k is a multiple of 4, at most QK_NORM_MAX_K; m below 2^24. Bit-exact. Device
 * pointers; float rows 16-byte aligned. The decode chain between two
 * matmuls: slm/qwen.c:936-948 (h = h + mix; ffn_norm) and the norm that
 * opens each layer's mixer (slm/qwen.c:332-334). */
#define QK_NORM_MAX_K 16384
int hip_add_rmsnorm_q8k(const float *h, const float *delta, const float *w,
                        float eps, int64_t m, int64_t k, float *h_out,
                        float *x_out, void *xq, void *stream);

/* y = x / (1 + expf(-x)) elementwise over n floats (y may equal x):
 * simd_silu_f32's x86 path (simd/simd.c:265-277) with expf bit for bit
 * the glibc expf that x86 hosts with FMA run. */
int hip_silu_f32(const float *x, int64_t n, float *y, void *stream);

/* The FFN's SwiGLU link (slm/qwen.c:949-954): act = silu(gate) * up over
 * m rows of k floats (simd_silu_f32 then tensor_mul, slm/tensor.c:293),
 * written to act (may be NULL) and/or quantized to Q8_K rows in xq (may
 * be NULL, needs k % 256 == 0) for the down projection; m*k at most
 * 2^33. Bit-exact. */
int hip_swiglu_q8k(const float *gate, const float *up, int64_t m, int64_t k,
                   float *act, void *xq, void *stream);

/* ---- device layer: LM head ------------------------------------------ */

/* Q6_K GEMV over n vocabulary rows fused with the greedy pick and a
 * top-k gather:
 *   logits (optional, may be NULL): n floats, as hip_matvec_q6k;
 *   *argmax: first index of the maximum logit (sample_argmax,
 *            slm/model.c:401-412: strict '>', NaN never wins);
 *   topk_idx/topk_val (optional when topk == 0): the set
 *            topk_collect (slm/sampler.c:70-93) keeps whenever the
 *            topk-th largest number is not tied: the topk largest logits,
 *            except that a NaN among the first topk rows keeps its slot
 *            (the rest are the largest numbers) and a NaN at row 0 keeps
 *            rows 0..topk-1; a later NaN never enters. Ranked numbers
 *            first, value-descending (ties by lower index), then the NaN
 *            rows by row.
 * 0 <= topk <= QK_TOPK_MAX. All outputs are device pointers.
 * Selection scratch is kept per stream: calls on different streams run
 * concurrently without sharing it. A stream's scratch is replaced (never
 * freed before hip_qk_shutdown) when a call needs more, so the first call
 * on a stream, and a first call with logits == NULL or a larger n,
 * allocate; later calls of the same or smaller size do not, and may be
 * captured in a HIP graph on that stream. A call that would allocate on a
 * stream that is capturing fails with QK_ERR_ARG and enqueues nothing
 * (hip_lmhead_q6k_argmax_topk_noalloc never allocates). */
#define QK_TOPK_MAX 256
int hip_lmhead_q6k_argmax_topk(const void *w, int64_t n, int64_t k,
                               const void *xq, int topk, float *logits,
                               int32_t *argmax, int32_t *topk_idx,
                               float *topk_val, void *stream);

/* The LM head above with no allocation at all, for callers that cannot
 * call hipMalloc: code under HIP graph capture, tight serving loops,
 * harnesses that forbid allocation. It has no counterpart in the
 * reference. Its selection scratch (and, when logits == NULL, the logits)
 * live in a static device array of each GPU, about 1.1 MB, held until the
 * process ends. With logits == NULL, n is at most QK_NOALLOC_MAX_N.
 * Every call on one GPU shares that array, whichever stream it uses:
 * calls that overlap in time on one GPU race, so keep them on one stream
 * or order them. An eager call from another stream while the previous
 * eager call is still in flight fails with QK_ERR_ARG and enqueues
 * nothing; calls captured into graphs are not tracked, so graphs that
 * hold this call must be replayed in order. Same arguments and results
 * as hip_lmhead_q6k_argmax_topk. */
#define QK_NOALLOC_MAX_N 262144
int hip_lmhead_q6k_argmax_topk_noalloc(const void *w, int64_t n, int64_t k,
                                       const void *xq, int topk,
                                       float *logits, int32_t *argmax,
                                       int32_t *topk_idx, float *topk_val,
                                       void *stream);

/* ---- device layer: sampler chain ------------------------------------ */

/* The fields of struct slm_sampler (slm/slm.h:117-124). */
typedef struct {
    float   temperature;        /* <= 0: greedy argmax                   */
    int32_t top_k;              /* <= 0: 256; capped at 256              */
    float   top_p;              /* (0, 1): nucleus; else off             */
    float   min_p;              /* > 0: drop below min_p * top prob      */
    float   repetition_penalty; /* 1: off                                */
    int32_t repetition_window;  /* <= 0: the whole history               */
} qk_sampler;

/* One sampling step of slm_generate_raw (slm/slm.c:309-324) on device
 * logits: the n_mask ids in mask (host array; eos / eot while fewer than
 * min_new tokens exist) are set to -inf, then sample_with
 * (slm/sampler.c:134-181): the repetition penalty over the last
 * repetition_window of history (device, hist_n ids), applied in place as
 * the reference does; with temperature <= 0 the first index of the
 * largest logit (sample_argmax); otherwise topk_collect, the temperature
 * softmax over its slots, the stable descending sort, top-p, min-p and
 * the roulette pick with one draw from the reference's rng, whose two
 * words (struct rng, slm/model.c:414) live in device memory at rng and
 * advance exactly as rng_next does. *token (device) receives the id.
 * After the pick the masked ids get back the values they had before
 * masking, as slm_generate_raw restores eos / eot after sample_with
 * (slm/slm.c:324-333; an id masked twice keeps the -inf the first mask
 * left); the other logits stay penalized. The pick, the logits and the
 * rng state are bit for bit the reference's, NaN logits included. token
 * may point into history (at entry hist_n) to append the pick. Scratch is
 * per stream, as for the LM head. n is at most QK_SAMPLE_MAX_N. */
#define QK_SAMPLE_MAX_MASK 2
#define QK_SAMPLE_MAX_N 262144
int hip_sample(float *logits, int64_t n, const qk_sampler *sp, uint64_t *rng,
               const int32_t *history, int32_t hist_n, const int32_t *mask,
               int32_t n_mask, int32_t *token, void *stream);

/* ---- device layer: chunked Gated DeltaNet prefill ------------------ */

/* The chunk loop of slm_forward_ssm_batch (slm/qwen.c:772-807) over one
 * layer: n_tok tokens in chunks of 64, each chunk run through
 * chunked_ssm_step_f32 (slm/chunked.c:287-521) for every head, the state
 * of each head carried from chunk to chunk. q, k: [n_tok][n_heads][k_hd]
 * (q L2-normalized and scaled, k L2-normalized); v: [n_tok][n_heads][v_hd];
 * g_log, beta: [n_tok][n_heads]; state: [n_heads][k_hd][v_hd], updated in
 * place; out: [n_tok][n_heads][v_hd]. Bit-exact against the reference's
 * x86 build (sequential fp32 sums, expf of glibc's FMA build). Head dims
 * at most QK_DELTANET_MAX_HD. Device pointers; out must not overlap the
 * inputs or the state (rejected); scratch per stream, as for the LM head. */
#define QK_DELTANET_MAX_HD 128
int hip_deltanet_chunked(const float *q, const float *k, const float *v,
                         const float *g_log, const float *beta, int64_t n_tok,
                         int n_heads, int k_hd, int v_hd, float *state,
                         float *out, void *stream);

/* ---- host seam ------------------------------------------------------ */

/* Upload the n x k weight matrix at host address `host_w` (GGUF type
 * `type`) once; later host-seam calls with the same address use the
 * device copy. Weights are immutable after load (slm/slm.h:12-13), so
 * re-registering an address is a no-op. Thread-safe. */
int hip_qk_register_weight(const void *host_w, int type, int64_t k,
                           int64_t n);
int hip_qk_unregister_weight(const void *host_w);
/* Drop every registered weight whose host bytes overlap
 * [base, base + bytes) and free its device copy; returns how many were
 * dropped (0 when libqk is not initialized). The host seam calls it
 * before the reference unmaps a GGUF file (gguf_close, slm/gguf.c:263),
 * so a model loaded later at the same addresses is uploaded afresh.
 * Waits for host-seam calls still using those weights. */
int hip_qk_unregister_range(const void *base, size_t bytes);
/* Device address of a registered weight (NULL if unknown). */
const void *hip_qk_device_weight(const void *host_w);

/* out[t*out_f + j] = row_dot(W row j, quant(x row t)): exactly what
 * tensor_matmul_q4k_f32 / _q5k_ / _q6k_ / _q8_0_ compute
 * (slm/tensor.c:827, 898, 1012, 952), for x of n_tok rows of k floats
 * in host memory and out in host memory. Registers the weight on first
 * use. Synchronous. Each host thread runs its calls on a stream of its
 * own (the reference's contexts are single-threaded, slm/slm.h:33-36), so
 * calls from several threads overlap on the GPU. */
int hip_qk_matmul_host(const void *host_w, int type, int64_t out_f,
                       int64_t k, const float *x, int64_t n_tok,
                       float *out);
/* chunked_ssm_step_f32 (slm/chunked.c:287) for one head and one chunk of
 * n <= 64 tokens, host buffers in and out, synchronous: the body the host
 * seam gives the reference's chunk step (its scratch arguments are not
 * needed). q, k: [n][k_hd]; v, out: [n][v_hd]; g_log, beta: [n];
 * state: [k_hd][v_hd], updated in place. */
int hip_qk_deltanet_host(int n, int k_hd, int v_hd, const float *q,
                         const float *k, const float *v, const float *g_log,
                         const float *beta, float *state, float *out);
/* The chunk loop of slm_forward_ssm_batch over one layer
 * (slm/qwen.c:772-807) from host buffers, synchronous: what
 * hip_deltanet_chunked computes, on the reference's own arrays. q, k:
 * Q_all, K_all [n_tok][n_heads][k_hd]; v: V_all [n_tok][n_heads][v_hd];
 * g_log, beta: g_log_all, beta_all [n_tok][n_heads]; state: the layer's
 * state_base [n_heads][k_hd][v_hd], updated in place; out: out_flat
 * [n_tok][n_heads][v_hd]. All staged at once: at most
 * QK_DELTANET_HOST_MAX_BYTES of them per call. */
#define QK_DELTANET_HOST_MAX_BYTES (4.0 * 1024 * 1024 * 1024)
int hip_qk_deltanet_layer_host(int64_t n_tok, int n_heads, int k_hd,
                               int v_hd, const float *q, const float *k,
                               const float *v, const float *g_log,
                               const float *beta, float *state, float *out);
/* LM head: matmul_dispatch(&W.output, h) (slm/qwen.c:976) followed by
 * sample_argmax (slm/model.c:401). logits (n floats) may be NULL when
 * only the token is needed; topk may be 0. Host pointers. */
int hip_qk_lmhead_host(const void *host_w, int64_t n, int64_t k,
                       const float *x, int topk, float *logits,
                       int32_t *argmax, int32_t *topk_idx,
                       float *topk_val);

#pragma GCC visibility pop

#ifdef __cplusplus
}
#endif

#endif /* QK_H */
