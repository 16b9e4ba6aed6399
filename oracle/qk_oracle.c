/*
 * qk_oracle.c -- CPU restatement of qwen.haiku's quantized matmul path.
 *
 * TEST INFRASTRUCTURE ONLY (see qk_oracle.h). Each function names the
 * reference lines it restates. The oracle is pinned three ways in
 * tests/test_oracle.py: against the reference compiled from its own
 * sources (oracle/_ref, when present), against the committed golden
 * vectors under tests/golden/, and against closed forms (exhaustive
 * fp16, brute-force int64 dots, scale-unpack round trips, quantizer
 * invariants).
 */
#include "qk_oracle.h"

#include <math.h>
#include <stddef.h>
#include <string.h>

#define QK_K  256
#define QK8_0 32

/* Block layouts: simd/quants.h:95-130 (fp16 fields as raw bits). */
typedef struct { float d; int8_t qs[QK_K]; int16_t bsums[QK_K / 16]; } o_q8k;
typedef struct { uint16_t d, dmin; uint8_t scales[12]; uint8_t qs[QK_K / 2]; } o_q4k;
typedef struct { uint16_t d, dmin; uint8_t scales[12]; uint8_t qh[QK_K / 8]; uint8_t qs[QK_K / 2]; } o_q5k;
typedef struct { uint8_t ql[QK_K / 2]; uint8_t qh[QK_K / 4]; int8_t scales[QK_K / 16]; uint16_t d; } o_q6k;
typedef struct { uint16_t d; int8_t qs[QK8_0]; } o_q8_0;

typedef char o_sz_q8k[sizeof(o_q8k) == 292 ? 1 : -1];
typedef char o_sz_q4k[sizeof(o_q4k) == 144 ? 1 : -1];
typedef char o_sz_q5k[sizeof(o_q5k) == 176 ? 1 : -1];
typedef char o_sz_q6k[sizeof(o_q6k) == 210 ? 1 : -1];
typedef char o_sz_q80[sizeof(o_q8_0) == 34 ? 1 : -1];

static uint32_t fbits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static float    bitsf(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* simd/quants.h:50-53: with clang, q_fp16_to_f32 is a `_Float16` cast,
 * i.e. exact IEEE binary16 -> binary32 widening (subnormals kept). */
float qko_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
    float r;
    if (e == 0) {
        r = (float)m * 0x1p-24f;                       /* exact */
        r = sign ? -r : r;
    } else if (e == 31) {
        r = bitsf(sign | 0x7f800000u | (m << 13));
    } else {
        r = bitsf(sign | ((e + 112u) << 23) | (m << 13));
    }
    return r;
}

/* simd/quants.h:53 and slm/tensor.c:940 (`(_Float16)d`): IEEE
 * binary32 -> binary16, round to nearest even, overflow to inf. */
uint16_t qko_f32_to_f16(float f) {
    uint32_t x = fbits(f);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7fffffffu;
    uint32_t q;
    if (ax > 0x7f800000u) {                            /* NaN: quiet  */
        q = 0x7e00u | ((ax >> 13) & 0x3ffu);
    } else if (ax >= 0x477ff000u) {                    /* >= 65520    */
        q = 0x7c00u;
    } else if (ax >= 0x38800000u) {                    /* fp16 normal */
        uint32_t rem = ax & 0x1fffu;
        q = (((ax >> 23) - 112u) << 10) | ((ax >> 13) & 0x3ffu);
        if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) q += 1;
    } else if (ax <= 0x33000000u) {                    /* <= 2^-25    */
        q = 0;
    } else {                                           /* subnormal   */
        uint32_t m = (ax & 0x7fffffu) | 0x800000u;
        uint32_t shift = 126u - (ax >> 23);            /* 14..24      */
        uint32_t rem = m & ((1u << shift) - 1u), half = 1u << (shift - 1);
        q = m >> shift;
        if (rem > half || (rem == half && (q & 1u))) q += 1;
    }
    return (uint16_t)(sign | q);
}

/* simd/quants.h:137-142, slm/tensor.c:673-678: magic-number rounding,
 * half to even for |v| < 2^22. The add is a separate rounding. */
int32_t qko_nearest_int(float v) {
    volatile float t = v + 12582912.f;
    int32_t i;
    float tt = t;
    memcpy(&i, &tt, 4);
    return (i & 0x007fffff) - 0x00400000;
}

/* slm/tensor.c:683-720 (= simd/quants.h:156-186). */
void qko_quantize_q8k(const float *x, void *xq, int64_t k) {
    o_q8k *y = (o_q8k *)xq;
    for (int64_t b = 0; b < k / QK_K; b++) {
        const float *s = x + b * QK_K;
        float amax = 0.0f, xmax = 0.0f;
        for (int i = 0; i < QK_K; i++) {
            float ax = fabsf(s[i]);
            if (ax > amax) { amax = ax; xmax = s[i]; }
        }
        if (amax == 0.0f) {
            y[b].d = 0.0f;
            memset(y[b].qs, 0, sizeof(y[b].qs));
            memset(y[b].bsums, 0, sizeof(y[b].bsums));
        } else {
            float iscale = -127.0f / xmax;
            y[b].d = 1.0f / iscale;
            for (int i = 0; i < QK_K; i++) {
                int32_t v = qko_nearest_int(iscale * s[i]);
                if (v > 127) v = 127;
                if (v < -128) v = -128;
                y[b].qs[i] = (int8_t)v;
            }
            for (int j = 0; j < QK_K / 16; j++) {
                int32_t acc = 0;
                for (int l = 0; l < 16; l++) acc += y[b].qs[j * 16 + l];
                y[b].bsums[j] = (int16_t)acc;
            }
        }
    }
}

/* slm/tensor.c:930-950: amax/127, reciprocal of the unrounded d,
 * roundf (half away from zero), d stored as fp16 RNE, clamp to int8. */
void qko_quantize_q8_0(const float *x, void *xq, int64_t k) {
    o_q8_0 *y = (o_q8_0 *)xq;
    for (int64_t i = 0; i < k / QK8_0; i++) {
        float amax = 0.0f;
        for (int j = 0; j < QK8_0; j++) {
            float v = fabsf(x[i * QK8_0 + j]);
            if (v > amax) amax = v;
        }
        float d = amax / 127.0f;
        float id = (d != 0.0f) ? (1.0f / d) : 0.0f;
        y[i].d = qko_f32_to_f16(d);
        for (int j = 0; j < QK8_0; j++) {
            /* (int32_t)roundf() of a value outside int32 is undefined in
             * C; the reference as compiled (clang -O3) saturates, which
             * shows when d underflows and id = 1/d is inf. */
            float r = roundf(x[i * QK8_0 + j] * id);
            int32_t q = r >= 127.0f ? 127 : (r <= -128.0f ? -128 : (int32_t)r);
            y[i].qs[j] = (int8_t)q;
        }
    }
}

/* simd/quants.h:215-224. */
void qko_scale_min(const uint8_t *s, int j, uint8_t *sc, uint8_t *m) {
    if (j < 4) {
        *sc = s[j] & 63;
        *m  = s[j + 4] & 63;
    } else {
        *sc = (uint8_t)((s[j + 4] & 0x0f) | ((s[j - 4] >> 6) << 4));
        *m  = (uint8_t)((s[j + 4] >> 4) | ((s[j] >> 6) << 4));
    }
}

/* Integer part of Q4_K . Q8_K for one super-block, simd/quants.h:
 * 283-304 (isum over 4 chunks of 64: low nibbles of qs[32c..] with
 * q8[64c..], high nibbles with q8[64c+32..]; isum_mins from bsum
 * pairs). */
void qko_q4k_block_ints(const void *wv, const void *xv, int32_t *isum,
                        int32_t *isum_mins) {
    const o_q4k *w = (const o_q4k *)wv;
    const o_q8k *y = (const o_q8k *)xv;
    uint8_t sc[8], mn[8];
    for (int j = 0; j < 8; j++) qko_scale_min(w->scales, j, &sc[j], &mn[j]);
    int32_t mins = 0;
    for (int j = 0; j < 8; j++)
        mins += ((int32_t)y->bsums[2 * j] + y->bsums[2 * j + 1]) * mn[j];
    int32_t acc = 0;
    for (int c = 0; c < 4; c++) {
        int32_t s1 = 0, s2 = 0;
        for (int l = 0; l < 32; l++) {
            s1 += (w->qs[32 * c + l] & 0x0f) * (int32_t)y->qs[64 * c + l];
            s2 += (w->qs[32 * c + l] >> 4) * (int32_t)y->qs[64 * c + 32 + l];
        }
        acc += s1 * sc[2 * c] + s2 * sc[2 * c + 1];
    }
    *isum = acc;
    *isum_mins = mins;
}

/* simd/quants.h:324-349: the 5th bit of element l of chunk c is bit 2c
 * (low half) / 2c+1 (high half) of qh[l]. */
void qko_q5k_block_ints(const void *wv, const void *xv, int32_t *isum,
                        int32_t *isum_mins) {
    const o_q5k *w = (const o_q5k *)wv;
    const o_q8k *y = (const o_q8k *)xv;
    uint8_t sc[8], mn[8];
    for (int j = 0; j < 8; j++) qko_scale_min(w->scales, j, &sc[j], &mn[j]);
    int32_t mins = 0;
    for (int j = 0; j < 8; j++)
        mins += ((int32_t)y->bsums[2 * j] + y->bsums[2 * j + 1]) * mn[j];
    int32_t acc = 0;
    for (int c = 0; c < 4; c++) {
        int32_t s1 = 0, s2 = 0;
        for (int l = 0; l < 32; l++) {
            int32_t lo = (w->qs[32 * c + l] & 0x0f) + (((w->qh[l] >> (2 * c)) & 1) << 4);
            int32_t hi = (w->qs[32 * c + l] >> 4) + (((w->qh[l] >> (2 * c + 1)) & 1) << 4);
            s1 += lo * (int32_t)y->qs[64 * c + l];
            s2 += hi * (int32_t)y->qs[64 * c + 32 + l];
        }
        acc += s1 * sc[2 * c] + s2 * sc[2 * c + 1];
    }
    *isum = acc;
    *isum_mins = mins;
}

/* Raw 6-bit weight of element e (0..255) of a Q6_K block, the index map
 * of simd/quants.h:370-394 / slm/tensor.c:994-1003: half h = e/128,
 * within it position p = e%128, quarter q = p/32, l = p%32; low nibble
 * from ql[64h + l + 32*(q&1)] (>>4 when q >= 2), high pair from
 * qh[32h + l] bits 2q..2q+1. */
static int32_t q6_raw(const o_q6k *w, int e) {
    int h = e / 128, p = e % 128, q = p / 32, l = p % 32;
    uint8_t lb = w->ql[64 * h + l + 32 * (q & 1)];
    int32_t lo = (q >= 2) ? (lb >> 4) : (lb & 0x0f);
    int32_t hi = (w->qh[32 * h + l] >> (2 * q)) & 3;
    return lo | (hi << 4);
}

/* simd/quants.h:359-399: isum over 16 sub-blocks of 16 with signed
 * scales, isum_mins = sum bsums[s]*scales[s]. */
void qko_q6k_block_ints(const void *wv, const void *xv, int32_t *isum,
                        int32_t *isum_mins) {
    const o_q6k *w = (const o_q6k *)wv;
    const o_q8k *y = (const o_q8k *)xv;
    int32_t mins = 0, acc = 0;
    for (int s = 0; s < 16; s++) mins += (int32_t)y->bsums[s] * w->scales[s];
    for (int s = 0; s < 16; s++) {
        int32_t part = 0;
        for (int l = 0; l < 16; l++)
            part += q6_raw(w, 16 * s + l) * (int32_t)y->qs[16 * s + l];
        acc += part * w->scales[s];
    }
    *isum = acc;
    *isum_mins = mins;
}

/* Float epilogue of Q4_K/Q5_K per super-block.
 * separate: simd/quants.h:305 and simd/avx.c:654 (AVX1), no FMA:
 *           rn(rn(d*isum) - rn(dmin*mins));
 * fused:    simd/avx.c:229,466,515 (AVX2/VNNI), contracted by clang to
 *           fma(d, isum, -rn(dmin*mins)).
 * d = rn(y.d * fp16(x.d)), dmin = rn(y.d * fp16(x.dmin)). */
static float k_term(float yd, uint16_t xd, uint16_t xdmin, int32_t isum,
                    int32_t mins, int epi) {
    float d = yd * qko_f16_to_f32(xd);
    float dmin = yd * qko_f16_to_f32(xdmin);
    float fi = (float)isum, fm = (float)mins;
    float t;
    if (epi == QKO_EPI_FUSED) {
        volatile float pm = dmin * fm;
        t = fmaf(d, fi, -pm);
    } else {
        volatile float a = d * fi;
        volatile float b = dmin * fm;
        t = a - b;
    }
    return t;
}

/* simd/avx.c:231-240 (and :300,:405,:467,:516,:587): the AVX2/VNNI
 * kernels accumulate the row sum broadcast in 8 lanes and return
 * hsum(8 lanes) / 8, i.e. ((s+s)+(s+s))+((s+s)+(s+s)) / 8. That equals s
 * unless 8s overflows, in which case it is +-inf. */
static float avx_bcast_sum(float s) {
    volatile float s2 = s + s;
    volatile float s4 = s2 + s2;
    volatile float s8 = s4 + s4;
    return s8 / 8.0f;
}

/* simd/quants.h:267-306 (separate) / simd/avx.c:420-468 (fused): the
 * row sum starts at 0 and adds one term per super-block in order (the
 * AVX2/VNNI 8-lane broadcast and /8 are exact). */
float qko_q4k_dot(int nb, const void *wv, const void *xv, int epi) {
    const o_q4k *w = (const o_q4k *)wv;
    const o_q8k *y = (const o_q8k *)xv;
    float sum = 0.0f;
    for (int i = 0; i < nb; i++) {
        int32_t is, im;
        qko_q4k_block_ints(&w[i], &y[i], &is, &im);
        sum += k_term(y[i].d, w[i].d, w[i].dmin, is, im, epi);
    }
    return epi == QKO_EPI_FUSED ? avx_bcast_sum(sum) : sum;
}

/* simd/quants.h:310-351 / simd/avx.c:470-523. */
float qko_q5k_dot(int nb, const void *wv, const void *xv, int epi) {
    const o_q5k *w = (const o_q5k *)wv;
    const o_q8k *y = (const o_q8k *)xv;
    float sum = 0.0f;
    for (int i = 0; i < nb; i++) {
        int32_t is, im;
        qko_q5k_block_ints(&w[i], &y[i], &is, &im);
        sum += k_term(y[i].d, w[i].d, w[i].dmin, is, im, epi);
    }
    return epi == QKO_EPI_FUSED ? avx_bcast_sum(sum) : sum;
}

/* simd/quants.h:399 and simd/avx.c:404,586,827: every tier computes
 * rn(rn(fp16(x.d) * y.d) * (float)(isum - 32*isum_mins)) per block and
 * sums in block order; AVX2/VNNI return it through the 8-lane broadcast. */
float qko_q6k_dot(int nb, const void *wv, const void *xv, int epi) {
    const o_q6k *w = (const o_q6k *)wv;
    const o_q8k *y = (const o_q8k *)xv;
    float sum = 0.0f;
    for (int i = 0; i < nb; i++) {
        int32_t is, im;
        qko_q6k_block_ints(&w[i], &y[i], &is, &im);
        volatile float s = qko_f16_to_f32(w[i].d) * y[i].d;
        volatile float t = s * (float)(is - 32 * im);
        sum += t;
    }
    return epi == QKO_EPI_FUSED ? avx_bcast_sum(sum) : sum;
}

/* separate: simd/quants.h:244-256 and simd/avx.c:136-158:
 *   sum += (float)sumi * rn(fp16(x.d)*fp16(y.d)) per block.
 * fused: simd/avx.c:65-123: lane l (l < 8) accumulates
 *   acc_l = fma((float)p_l, s_b, acc_l), p_l the 4-byte partial dot of
 *   bytes 4l..4l+3 of block b, then the reduction tree
 *   ((a0+a4)+(a1+a5)) + ((a2+a6)+(a3+a7)). */
float qko_q8_0_dot(int64_t k, const void *wv, const void *xv, int epi) {
    const o_q8_0 *x = (const o_q8_0 *)wv;
    const o_q8_0 *y = (const o_q8_0 *)xv;
    int64_t nb = k / QK8_0;
    float r;
    if (epi == QKO_EPI_FUSED) {
        float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        for (int64_t i = 0; i < nb; i++) {
            volatile float s = qko_f16_to_f32(x[i].d) * qko_f16_to_f32(y[i].d);
            for (int l = 0; l < 8; l++) {
                int32_t p = 0;
                for (int b = 0; b < 4; b++)
                    p += (int32_t)x[i].qs[4 * l + b] * y[i].qs[4 * l + b];
                acc[l] = fmaf((float)p, s, acc[l]);
            }
        }
        volatile float s04 = acc[0] + acc[4], s15 = acc[1] + acc[5];
        volatile float s26 = acc[2] + acc[6], s37 = acc[3] + acc[7];
        volatile float lo = s04 + s15, hi = s26 + s37;
        r = lo + hi;
    } else {
        float sum = 0.0f;
        for (int64_t i = 0; i < nb; i++) {
            int32_t p = 0;
            for (int j = 0; j < QK8_0; j++) p += (int32_t)x[i].qs[j] * y[i].qs[j];
            volatile float s = qko_f16_to_f32(x[i].d) * qko_f16_to_f32(y[i].d);
            volatile float t = (float)p * s;
            sum += t;
        }
        r = sum;
    }
    return r;
}

/* slm/tensor.c:800-820: y = rn(rn(d1*q) - m1), d1 = rn(d*sc),
 * m1 = rn(dmin*m). The x86 host build has no FMA to contract into. */
void qko_dequant_q4k(const void *wv, int64_t nblocks, float *out) {
    const o_q4k *w = (const o_q4k *)wv;
    for (int64_t b = 0; b < nblocks; b++) {
        const float d = qko_f16_to_f32(w[b].d), mn = qko_f16_to_f32(w[b].dmin);
        float *y = out + b * QK_K;
        for (int c = 0; c < 4; c++) {
            uint8_t sc, m;
            qko_scale_min(w[b].scales, 2 * c, &sc, &m);
            volatile float d1 = d * (float)sc, m1 = mn * (float)m;
            qko_scale_min(w[b].scales, 2 * c + 1, &sc, &m);
            volatile float d2 = d * (float)sc, m2 = mn * (float)m;
            for (int l = 0; l < 32; l++) {
                volatile float a = d1 * (float)(w[b].qs[32 * c + l] & 0x0f);
                volatile float e = d2 * (float)(w[b].qs[32 * c + l] >> 4);
                y[64 * c + l] = a - m1;
                y[64 * c + 32 + l] = e - m2;
            }
        }
    }
}

/* slm/tensor.c:867-896. */
void qko_dequant_q5k(const void *wv, int64_t nblocks, float *out) {
    const o_q5k *w = (const o_q5k *)wv;
    for (int64_t b = 0; b < nblocks; b++) {
        const float d = qko_f16_to_f32(w[b].d), mn = qko_f16_to_f32(w[b].dmin);
        float *y = out + b * QK_K;
        for (int c = 0; c < 4; c++) {
            uint8_t sc, m;
            qko_scale_min(w[b].scales, 2 * c, &sc, &m);
            volatile float d1 = d * (float)sc, m1 = mn * (float)m;
            qko_scale_min(w[b].scales, 2 * c + 1, &sc, &m);
            volatile float d2 = d * (float)sc, m2 = mn * (float)m;
            for (int l = 0; l < 32; l++) {
                int32_t lo = (w[b].qs[32 * c + l] & 0x0f) + (((w[b].qh[l] >> (2 * c)) & 1) << 4);
                int32_t hi = (w[b].qs[32 * c + l] >> 4) + (((w[b].qh[l] >> (2 * c + 1)) & 1) << 4);
                volatile float a = d1 * (float)lo, e = d2 * (float)hi;
                y[64 * c + l] = a - m1;
                y[64 * c + 32 + l] = e - m2;
            }
        }
    }
}

/* slm/tensor.c:988-1010: y = rn(rn(d*sc) * (u6 - 32)). */
void qko_dequant_q6k(const void *wv, int64_t nblocks, float *out) {
    const o_q6k *w = (const o_q6k *)wv;
    for (int64_t b = 0; b < nblocks; b++) {
        const float d = qko_f16_to_f32(w[b].d);
        for (int e = 0; e < QK_K; e++) {
            volatile float ds = d * (float)w[b].scales[e / 16];
            out[b * QK_K + e] = ds * (float)(q6_raw(&w[b], e) - 32);
        }
    }
}

static int type_block(int type, int64_t *elems, int64_t *bytes) {
    int ok = 1;
    switch (type) {
        case 8:  *elems = QK8_0; *bytes = sizeof(o_q8_0); break;
        case 12: *elems = QK_K;  *bytes = sizeof(o_q4k);  break;
        case 13: *elems = QK_K;  *bytes = sizeof(o_q5k);  break;
        case 14: *elems = QK_K;  *bytes = sizeof(o_q6k);  break;
        default: ok = 0; break;
    }
    return ok;
}

/* slm/tensor.c:838-851 (and 908-918, 968-980, 1022-1032): per token t,
 * out[t*n + j] = row_dot(W row j, xq row t). */
int qko_matmul_xq(int type, const void *w, int64_t n, int64_t k,
                  const void *xq, int64_t m, float *out, int epi,
                  int64_t row0, int64_t row1) {
    int64_t be, bb;
    if (!type_block(type, &be, &bb) || k % be) return -1;
    const int64_t nb = k / be;
    const int64_t xbytes = (type == 8) ? (int64_t)sizeof(o_q8_0) : (int64_t)sizeof(o_q8k);
    for (int64_t t = 0; t < m; t++) {
        const char *xr = (const char *)xq + t * nb * xbytes;
        for (int64_t j = row0; j < row1; j++) {
            const char *wr = (const char *)w + j * nb * bb;
            float v;
            switch (type) {
                case 8:  v = qko_q8_0_dot(k, wr, xr, epi); break;
                case 12: v = qko_q4k_dot((int)nb, wr, xr, epi); break;
                case 13: v = qko_q5k_dot((int)nb, wr, xr, epi); break;
                default: v = qko_q6k_dot((int)nb, wr, xr, epi); break;
            }
            out[t * n + j] = v;
        }
    }
    return 0;
}

int qko_matmul(int type, const void *w, int64_t n, int64_t k,
               const float *x, int64_t m, float *out, int epi,
               int64_t row0, int64_t row1) {
    int64_t be, bb;
    if (!type_block(type, &be, &bb) || k % be) return -1;
    /* One quantized activation row at a time, as the reference does. */
    static __thread unsigned char buf[(1 << 16) / 256 * 292 + 64];
    const int64_t xbytes = (type == 8) ? (k / QK8_0) * 34 : (k / QK_K) * 292;
    if (xbytes > (int64_t)sizeof(buf)) return -2;
    for (int64_t t = 0; t < m; t++) {
        if (type == 8) qko_quantize_q8_0(x + t * k, buf, k);
        else           qko_quantize_q8k(x + t * k, buf, k);
        int r = qko_matmul_xq(type, w, n, k, buf, 1, out + t * n, epi, row0, row1);
        if (r) return r;
    }
    return 0;
}

/* slm/model.c:401-412: first index of the maximum, strict '>'. */
int32_t qko_argmax(const float *v, int64_t n) {
    int32_t best = 0;
    float b = v[0];
    for (int64_t i = 1; i < n; i++) {
        if (v[i] > b) { b = v[i]; best = (int32_t)i; }
    }
    return best;
}

/* slm/sampler.c:70-93: fill k slots in scan order, then replace the
 * first minimum slot when strictly greater. */
int32_t qko_topk_collect(const float *v, int64_t n, int32_t k,
                         int32_t *idx, float *val) {
    int32_t filled = 0;
    if (k <= 0 || k > 256) k = 256;
    for (int64_t i = 0; i < n; i++) {
        if (filled < k) {
            idx[filled] = (int32_t)i;
            val[filled] = v[i];
            filled++;
        } else {
            int32_t worst = 0;
            for (int32_t j = 1; j < k; j++)
                if (val[j] < val[worst]) worst = j;
            if (v[i] > val[worst]) { idx[worst] = (int32_t)i; val[worst] = v[i]; }
        }
    }
    return filled;
}

/* ---- the decode chain's elementwise links ---------------------------- */

/* tensor_add (slm/tensor.c:284-291) of an optional delta, then
 * tensor_rms_norm (slm/tensor.c:345-367) per row of k floats: a
 * sequential double sum of the float squares, then
 * rscale = 1/sqrtf((float)(ssq/k) + eps), x = (r*rscale)*w. */
void qko_add_rmsnorm(const float *h, const float *delta, const float *w,
                     float eps, int64_t m, int64_t k, float *h_out,
                     float *x_out) {
    for (int64_t t = 0; t < m; t++) {
        const float *hr = h + t * k;
        const float *dr = delta ? delta + t * k : NULL;
        float *ro = h_out + t * k;
        for (int64_t i = 0; i < k; i++) ro[i] = dr ? hr[i] + dr[i] : hr[i];
        double ssq = 0.0;
        for (int64_t i = 0; i < k; i++) {
            float sq = ro[i] * ro[i];
            ssq += (double)sq;
        }
        float mean = (float)(ssq / (double)k);
        float rscale = 1.0f / sqrtf(mean + eps);
        float *xo = x_out + t * k;
        for (int64_t i = 0; i < k; i++) {
            float a = ro[i] * rscale;
            xo[i] = a * w[i];
        }
    }
}

/* simd_silu_f32's x86 path (simd/simd.c:265-269) with the host libm. */
void qko_silu(int64_t n, const float *x, float *y) {
    for (int64_t i = 0; i < n; i++) {
        float v = x[i];
        float den = 1.0f + expf(-v);
        y[i] = v / den;
    }
}

/* silu(gate) then tensor_mul (slm/tensor.c:293-300) by up
 * (slm/qwen.c:949-954). */
void qko_swiglu(int64_t n, const float *gate, const float *up, float *act) {
    for (int64_t i = 0; i < n; i++) {
        float v = gate[i];
        float s = v / (1.0f + expf(-v));
        act[i] = s * up[i];
    }
}

/* ---- the sampler chain ------------------------------------------------ */

/* xoroshiro128-style step and uniform draw of the reference
 * (slm/model.c:414-447). */
static uint64_t o_rotl(uint64_t x, int k) { return (x << k) | (x >> (64 - k)); }

static uint64_t o_rng_next(uint64_t *st) {
    uint64_t s0 = st[0], s1 = st[1];
    uint64_t out = o_rotl(s0 * 5, 7) * 9;
    s1 ^= s0;
    st[0] = o_rotl(s0, 24) ^ s1 ^ (s1 << 16);
    st[1] = o_rotl(s1, 37);
    return out;
}

static float o_rng_uniform(uint64_t *st) {
    return (float)(o_rng_next(st) >> 40) / (float)(1u << 24);
}

/* The rng state slm_ctx_create / slm_generate_raw seed from one 64-bit
 * value (SplitMix64, slm/model.c:431-442). */
void qko_rng_seed(uint64_t seed, uint64_t *st) {
    uint64_t z = seed + 0x9e3779b97f4a7c15ULL;
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ULL;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebULL;
    st[0] = z ^ (z >> 31);
    z = st[0] + 0x9e3779b97f4a7c15ULL;
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ULL;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebULL;
    st[1] = z ^ (z >> 31);
    if (st[0] == 0 && st[1] == 0) st[0] = 1;
}

/* sample_with (slm/sampler.c:134-181): repetition penalty in place
 * (:49-63), greedy argmax when temperature <= 0, else topk_collect
 * (:70-93), topk_softmax (:97-111), topk_sort_desc (:116-129), top-p,
 * min-p and the roulette pick with one uniform draw. logits are modified
 * in place; st (2 words) advances on the sampling path only. */
static int32_t sample_with_core(float *logits, int64_t n, float temperature, int32_t top_k, float top_p,
                                float min_p, float penalty, int32_t window, uint64_t *st, const int32_t *history,
                                int32_t hist_n) {
    if (penalty != 1.0f && hist_n != 0) {
        int32_t start = (window > 0 && window < hist_n) ? hist_n - window : 0;
        for (int32_t i = start; i < hist_n; i++) {
            int32_t t = history[i];
            if (t >= 0 && (int64_t)t < n) {
                float lv = logits[t];
                logits[t] = lv > 0.0f ? lv / penalty : lv * penalty;
            }
        }
    }
    if (temperature <= 0.0f) return qko_argmax(logits, n);
    int32_t idx[256];
    float val[256];
    int32_t k = top_k > 0 ? top_k : 256;
    if (k > 256) k = 256;
    int32_t filled = qko_topk_collect(logits, n, k, idx, val);
    /* softmax over the survivors */
    float m = val[0];
    for (int32_t j = 1; j < filled; j++)
        if (val[j] > m) m = val[j];
    float sum = 0.0f;
    for (int32_t j = 0; j < filled; j++) {
        float z = (val[j] - m) / temperature;
        val[j] = expf(z);
        sum += val[j];
    }
    if (sum > 0.0f)
        for (int32_t j = 0; j < filled; j++) val[j] /= sum;
    /* stable descending insertion sort */
    for (int32_t i = 1; i < filled; i++) {
        float v = val[i];
        int32_t id = idx[i], j = i - 1;
        while (j >= 0 && val[j] < v) {
            val[j + 1] = val[j];
            idx[j + 1] = idx[j];
            j--;
        }
        val[j + 1] = v;
        idx[j + 1] = id;
    }
    int32_t cutoff = filled;
    if (top_p > 0.0f && top_p < 1.0f) {
        float acc = 0.0f;
        for (int32_t j = 0; j < filled; j++) {
            acc += val[j];
            if (acc >= top_p) { cutoff = j + 1; break; }
        }
    }
    if (min_p > 0.0f) {
        float thresh = min_p * val[0];
        int32_t j = 1;
        while (j < cutoff && val[j] >= thresh) j++;
        cutoff = j;
    }
    float tot = 0.0f;
    for (int32_t j = 0; j < cutoff; j++) tot += val[j];
    float u = o_rng_uniform(st) * tot;
    float c = 0.0f;
    int32_t picked = 0;
    for (int32_t j = 0; j < cutoff; j++) {
        c += val[j];
        if (u <= c) { picked = j; break; }
    }
    return idx[picked];
}

/* One sampling step of slm_generate_raw (slm/slm.c:309-333): each id in
 * mask (eos / eot while fewer than min_new tokens exist) has its value
 * saved and is set to -inf, in mask order; then sample_with; then the
 * saved values go back in mask order, so an id masked twice ends at the
 * second save, -inf. */
int32_t qko_sample(float *logits, int64_t n, float temperature, int32_t top_k, float top_p, float min_p,
                   float penalty, int32_t window, uint64_t *st, const int32_t *history, int32_t hist_n,
                   const int32_t *mask, int32_t n_mask) {
    float saved[n_mask > 0 ? n_mask : 1];
    for (int32_t i = 0; i < n_mask; i++)
        if (mask[i] >= 0 && mask[i] < n) {
            saved[i] = logits[mask[i]];
            logits[mask[i]] = -INFINITY;
        }
    const int32_t tok = sample_with_core(logits, n, temperature, top_k, top_p, min_p, penalty, window, st, history,
                                         hist_n);
    for (int32_t i = 0; i < n_mask; i++)
        if (mask[i] >= 0 && mask[i] < n) logits[mask[i]] = saved[i];
    return tok;
}

/* ---- chunked Gated DeltaNet ------------------------------------------- */

/* One chunk of n <= 64 tokens of one head (chunked_ssm_step_f32,
 * slm/chunked.c:287-521, on an x86 host: every dot and axpy is a
 * sequential mul-then-add, no FMA). q, k: [n][k_hd]; v: [n][v_hd];
 * g, beta: [n]; state [k_hd][v_hd] updated in place; out [n][v_hd]. */
void qko_chunked_step(int n, int kd, int vd, const float *q, const float *k, const float *v, const float *g,
                      const float *beta, float *state, float *out) {
    float gcs[64], gexp[64], dm[64 * 64], kb[64 * 128], vb[64 * 128], kkd[64 * 64], lhs[64 * 64];
    float attn[64 * 64], x[64 * 64], veff[64 * 128], kbg[64 * 128], kcd[64 * 128], akq[64 * 64];
    float qg[64 * 128], ainter[64 * 128], vnew[64 * 128];
    float run = 0.0f;
    for (int t = 0; t < n; t++) { run += g[t]; gcs[t] = run; }
    for (int t = 0; t < n; t++) gexp[t] = expf(gcs[t]);
    for (int i = 0; i < n; i++)
        for (int j = 0; j < n; j++) dm[i * n + j] = i > j ? expf(gcs[i] - gcs[j]) : 0.0f;
    for (int t = 0; t < n; t++) {
        for (int d = 0; d < kd; d++) kb[t * kd + d] = k[t * kd + d] * beta[t];
        for (int e = 0; e < vd; e++) vb[t * vd + e] = v[t * vd + e] * beta[t];
    }
    /* strictly lower: (K_j . Kbeta_i) * decay; lhs = I + that */
    for (int i = 0; i < n; i++)
        for (int j = 0; j < n; j++) {
            float val = 0.0f;
            if (i > j) {
                float s = 0.0f;
                for (int d = 0; d < kd; d++) s += k[j * kd + d] * kb[i * kd + d];
                val = s * dm[i * n + j];
            }
            kkd[i * n + j] = val;
            lhs[i * n + j] = i > j ? val : (i == j ? 1.0f : 0.0f);
        }
    for (int i = 0; i < n * n; i++) attn[i] = -kkd[i];
    /* forward substitution, column by column (ggml's solve_tri order) */
    for (int j = 0; j < n; j++)
        for (int i = 0; i < n; i++) {
            float s = 0.0f;
            for (int t = 0; t < i; t++) s += lhs[i * n + t] * x[t * n + j];
            x[i * n + j] = (attn[i * n + j] - s) / lhs[i * n + i];
        }
    for (int i = 0; i < n; i++)
        for (int j = 0; j < n; j++) attn[i * n + j] = j < i ? x[i * n + j] : (j == i ? 1.0f : 0.0f);
    /* attn @ v_beta, attn @ (k_beta * gexp): nonzero coefficients, j ascending */
    for (int t = 0; t < n; t++) for (int d = 0; d < kd; d++) kbg[t * kd + d] = kb[t * kd + d] * gexp[t];
    for (int i = 0; i < n; i++) {
        for (int e = 0; e < vd; e++) veff[i * vd + e] = 0.0f;
        for (int d = 0; d < kd; d++) kcd[i * kd + d] = 0.0f;
        for (int j = 0; j <= i; j++) {
            const float a = attn[i * n + j];
            if (a == 0.0f) continue;
            for (int e = 0; e < vd; e++) veff[i * vd + e] += a * vb[j * vd + e];
        }
        for (int j = 0; j <= i; j++) {
            const float a = attn[i * n + j];
            if (a == 0.0f) continue;
            for (int d = 0; d < kd; d++) kcd[i * kd + d] += a * kbg[j * kd + d];
        }
    }
    /* intra-chunk attention (K_j . Q_i) * decay, decay 1 on the diagonal */
    for (int i = 0; i < n; i++)
        for (int j = 0; j < n; j++) {
            float val = 0.0f;
            if (i >= j) {
                float s = 0.0f;
                for (int d = 0; d < kd; d++) s += k[j * kd + d] * q[i * kd + d];
                val = s * (i == j ? 1.0f : dm[i * n + j]);
            }
            akq[i * n + j] = val;
        }
    for (int t = 0; t < n; t++) for (int d = 0; d < kd; d++) qg[t * kd + d] = gexp[t] * q[t * kd + d];
    /* the carried state: state^T (q*gexp), state^T k_cumdecay; zero coefficients skipped */
    for (int t = 0; t < n; t++) {
        float vp[128];
        for (int e = 0; e < vd; e++) { ainter[t * vd + e] = 0.0f; vp[e] = 0.0f; }
        for (int d = 0; d < kd; d++) {
            const float c = qg[t * kd + d];
            if (c == 0.0f) continue;
            for (int e = 0; e < vd; e++) ainter[t * vd + e] += c * state[d * vd + e];
        }
        for (int d = 0; d < kd; d++) {
            const float c = kcd[t * kd + d];
            if (c == 0.0f) continue;
            for (int e = 0; e < vd; e++) vp[e] += c * state[d * vd + e];
        }
        for (int e = 0; e < vd; e++) vnew[t * vd + e] = veff[t * vd + e] - vp[e];
    }
    for (int t = 0; t < n; t++)
        for (int e = 0; e < vd; e++) {
            float s = 0.0f;
            for (int u = 0; u < n; u++) s += akq[t * n + u] * vnew[u * vd + e];
            out[t * vd + e] = ainter[t * vd + e] + s;
        }
    /* state := state * exp(g_last) + (K * exp(g_last - gcs))^T v_new */
    const float glast = gcs[n - 1], gle = expf(glast);
    float diff[64];
    for (int t = 0; t < n; t++) diff[t] = expf(glast - gcs[t]);
    for (int d = 0; d < kd; d++)
        for (int e = 0; e < vd; e++) {
            float s = 0.0f;
            for (int t = 0; t < n; t++) {
                const float kg = k[t * kd + d] * diff[t];
                s += kg * vnew[t * vd + e];
            }
            const float decayed = state[d * vd + e] * gle;
            state[d * vd + e] = decayed + s;
        }
}

/* slm_forward_ssm_batch's chunk loop (slm/qwen.c:772-807): n_tok tokens
 * in chunks of 64, every head per chunk, the state of each head carried.
 * q, k: [n_tok][n_heads][kd]; v, out: [n_tok][n_heads][vd]; g, beta:
 * [n_tok][n_heads]; state: [n_heads][kd][vd]. */
void qko_deltanet_chunked(int64_t n_tok, int n_heads, int kd, int vd, const float *q, const float *k,
                          const float *v, const float *g, const float *beta, float *state, float *out) {
    float qc[64 * 128], kc[64 * 128], vc[64 * 128], gc[64], bc[64], oc[64 * 128];
    for (int64_t c0 = 0; c0 < n_tok; c0 += 64) {
        const int n = (int)(n_tok - c0 < 64 ? n_tok - c0 : 64);
        for (int h = 0; h < n_heads; h++) {
            for (int t = 0; t < n; t++) {
                const int64_t tg = c0 + t;
                memcpy(qc + t * kd, q + (tg * n_heads + h) * kd, (size_t)kd * 4);
                memcpy(kc + t * kd, k + (tg * n_heads + h) * kd, (size_t)kd * 4);
                memcpy(vc + t * vd, v + (tg * n_heads + h) * vd, (size_t)vd * 4);
                gc[t] = g[tg * n_heads + h];
                bc[t] = beta[tg * n_heads + h];
            }
            qko_chunked_step(n, kd, vd, qc, kc, vc, gc, bc, state + (int64_t)h * kd * vd, oc);
            for (int t = 0; t < n; t++) memcpy(out + ((c0 + t) * n_heads + h) * vd, oc + t * vd, (size_t)vd * 4);
        }
    }
}
