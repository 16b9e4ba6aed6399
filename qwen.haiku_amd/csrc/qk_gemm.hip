// qk_gemm.hip -- chunked-prefill GEMM over native GGUF K-quant blocks
// (gfx950, int8 MFMA).
//
// y[t*n + j] = row_dot(W row j, xq row t): the token loop of
// tensor_matmul_q{4k,5k,6k}_f32 (slm/tensor.c:838-851, 908-918,
// 1022-1032) as one GEMM. Every output is bit-identical to the reference
// row dot of the selected tier, because the arithmetic is the same:
//
//  * per super-block, the integer dot of every sub-block is exact in
//    int32 (MFMA accumulate), multiplied by its sub-block scale and summed
//    in int32 (exact; the reference's order of integer adds is irrelevant);
//  * the super-block's float term is formed with the reference's rounding
//    sequence (separate or fused, as in the GEMV) and added to a running
//    fp32 sum in super-block order, exactly like the reference's
//    sequential `sum += term`.
//
// Work decomposition: a 256-thread workgroup owns a 64-token x 64-row
// output tile and walks the super-blocks of K in order. For each one it
// stages the 64 activation rows (int8 Q8_K quants, scale, bsum pairs)
// and the 64 weight rows, dequantised to int8 with their sub-block
// scales, into LDS; each of the 4 waves then computes a 32x32 sub-tile:
//
//  * Q4_K / Q5_K: one v_mfma_i32_32x32x32_i8 per 32-element sub-block
//    (weights 0..15 / 0..31), times the 6-bit scale; mins from the Q8_K
//    bsums (simd/quants.h:283-304, 324-349);
//  * Q6_K: one v_mfma_i32_32x32x16_i8 per 16-element sub-block, weights
//    staged as u6 - 32 in [-32, 31] so the reference's
//    isum - 32*isum_mins (simd/quants.h:359-399) is one exact int32 sum.
//
// The k-to-register order inside an MFMA is the hardware's; it is the
// same for both operands (each lane supplies 16 or 8 consecutive k of its
// row), so every product pairs the right weight with the right
// activation whatever that order is.
#include "qk_dev.h"
#include "qk_kernels.h"

namespace qk {

typedef int32_t v4i __attribute__((ext_vector_type(4)));
typedef int32_t v16i __attribute__((ext_vector_type(16)));

#define GM_BM 64                      // tokens per workgroup tile
#define GM_BN 64                      // weight rows per workgroup tile
#define GM_LD 272                     // LDS row stride of the int8 tiles (256 + 16)

struct __attribute__((aligned(16))) GemmLds {
    int8_t a[GM_BM][GM_LD];           // activation quants of the super-block
    int8_t b[GM_BN][GM_LD];           // dequantised int8 weights
    float yd[GM_BM];                  // Q8_K d per token
    int16_t bp[GM_BM][8];             // bsum pairs (bsums[2j] + bsums[2j+1])
    int8_t sc[GM_BN][16];             // sub-block scales per weight row
    uint8_t mn[GM_BN][8];             // 6-bit mins (Q4_K / Q5_K)
    float wd[GM_BN];                  // fp16 d, widened
    float wdm[GM_BN];                 // fp16 dmin, widened
};

__device__ __forceinline__ void lds_st16(void *p, uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
    *(QK_LDS uint4 *)p = make_uint4(a, b, c, d);
}

// ---- activation stage: tokens [t0, t0+64) of super-block i ---------------
__device__ __forceinline__ void stage_act(GemmLds &s, const uint8_t *__restrict__ xq, int64_t m, int nb,
                                          int64_t t0, int i) {
    for (int idx = threadIdx.x; idx < GM_BM * 73; idx += 256) {
        const int t = idx / 73, r = idx - t * 73;
        uint32_t v = 0;
        if (t0 + t < m) v = ld32(xq + ((t0 + t) * nb + i) * Q8K_BYTES + 4 * r);
        if (r == 0) {
            s.yd[t] = __uint_as_float(v);
        } else if (r <= 64) {
            *(QK_LDS uint32_t *)&s.a[t][4 * (r - 1)] = v;
        } else {
            s.bp[t][r - 65] = (int16_t)((int32_t)(int16_t)(v & 0xffffu) + (int32_t)(int16_t)(v >> 16));
        }
    }
}

// ---- weight stage: rows [r0, r0+64) of super-block i, dequantised ---------
// Q4_K (144 B = 9 x 16 B): piece 0 is d | dmin | scales, pieces 1..8 are
// qs; qs[32c + l] low nibble -> element 64c + l, high -> 64c + 32 + l.
__device__ __forceinline__ void stage_w_q4k(GemmLds &s, const uint8_t *__restrict__ w, int64_t n, int nb,
                                            int64_t r0, int i) {
    for (int idx = threadIdx.x; idx < GM_BN * 9; idx += 256) {
        const int r = idx / 9, p = idx - r * 9;
        const bool ok = r0 + r < n;
        const uint8_t *blk = w + ((r0 + r) * nb + i) * Q4K_BYTES;
        uint4 v = make_uint4(0, 0, 0, 0);
        if (ok) v = ld16(blk + 16 * p);
        if (p == 0) {
            int32_t sc, mm;
#pragma unroll
            for (int j = 0; j < 8; j++) {
                scale_min(v.y, v.z, v.w, j, sc, mm);
                s.sc[r][j] = (int8_t)sc;
                s.mn[r][j] = (uint8_t)mm;
            }
            s.wd[r] = h2f(v.x & 0xffffu);
            s.wdm[r] = h2f(v.x >> 16);
        } else {
            const int c = (p - 1) >> 1, l0 = 16 * ((p - 1) & 1);
            const uint32_t M = 0x0F0F0F0Fu;
            lds_st16(&s.b[r][64 * c + l0], v.x & M, v.y & M, v.z & M, v.w & M);
            lds_st16(&s.b[r][64 * c + 32 + l0], (v.x >> 4) & M, (v.y >> 4) & M, (v.z >> 4) & M, (v.w >> 4) & M);
        }
    }
}

// Q5_K (176 B = 11 x 16 B): piece 0 header, pieces 1-2 qh[32], pieces
// 3..10 qs. Element 64c + l gets bit 2c of qh[l] as its 5th bit, element
// 64c + 32 + l bit 2c+1.
__device__ __forceinline__ void stage_w_q5k(GemmLds &s, const uint8_t *__restrict__ w, int64_t n, int nb,
                                            int64_t r0, int i) {
    for (int idx = threadIdx.x; idx < GM_BN * 9; idx += 256) {
        const int r = idx / 9, p = idx - r * 9;
        const bool ok = r0 + r < n;
        const uint8_t *blk = w + ((r0 + r) * nb + i) * Q5K_BYTES;
        if (p == 0) {
            uint4 v = make_uint4(0, 0, 0, 0);
            if (ok) v = ld16(blk);
            int32_t sc, mm;
#pragma unroll
            for (int j = 0; j < 8; j++) {
                scale_min(v.y, v.z, v.w, j, sc, mm);
                s.sc[r][j] = (int8_t)sc;
                s.mn[r][j] = (uint8_t)mm;
            }
            s.wd[r] = h2f(v.x & 0xffffu);
            s.wdm[r] = h2f(v.x >> 16);
        } else {
            const int c = (p - 1) >> 1, half = (p - 1) & 1, l0 = 16 * half;
            uint4 q = make_uint4(0, 0, 0, 0), h = make_uint4(0, 0, 0, 0);
            if (ok) {
                q = ld16(blk + 48 + 16 * (p - 1));
                h = ld16(blk + 16 + 16 * half);
            }
            const uint32_t M = 0x0F0F0F0Fu, B1 = 0x01010101u;
            const uint32_t s0 = 2 * c, s1 = 2 * c + 1;
            lds_st16(&s.b[r][64 * c + l0], (q.x & M) | (((h.x >> s0) & B1) << 4), (q.y & M) | (((h.y >> s0) & B1) << 4),
                     (q.z & M) | (((h.z >> s0) & B1) << 4), (q.w & M) | (((h.w >> s0) & B1) << 4));
            lds_st16(&s.b[r][64 * c + 32 + l0], ((q.x >> 4) & M) | (((h.x >> s1) & B1) << 4),
                     ((q.y >> 4) & M) | (((h.y >> s1) & B1) << 4), ((q.z >> 4) & M) | (((h.z >> s1) & B1) << 4),
                     ((q.w >> 4) & M) | (((h.w >> s1) & B1) << 4));
        }
    }
}

// 16 bytes at a 2-byte aligned address inside a block, read as five
// aligned dwords and funnel-shifted (the last dword read ends at most 4
// bytes past the 16, which callers keep inside the block).
__device__ __forceinline__ uint4 ld16_a2(const uint8_t *p) {
    const uint32_t sh = (uint32_t)reinterpret_cast<uintptr_t>(p) & 3u;
    const uint8_t *a = p - sh;
    const uint32_t d0 = ld32(a), d1 = ld32(a + 4), d2 = ld32(a + 8), d3 = ld32(a + 12), d4 = ld32(a + 16);
    return make_uint4(__builtin_amdgcn_alignbyte(d1, d0, sh), __builtin_amdgcn_alignbyte(d2, d1, sh),
                      __builtin_amdgcn_alignbyte(d3, d2, sh), __builtin_amdgcn_alignbyte(d4, d3, sh));
}

// Four bytes u6 in [0, 63] -> four int8 bytes u6 - 32. u6 ^ 0x20 is
// u6 - 32 as a 6-bit two's-complement number (bit 5 the sign); copying
// bit 5 into bits 6 and 7 sign-extends it to 8 bits, byte by byte.
__device__ __forceinline__ uint32_t u6_minus_32(uint32_t x) {
    const uint32_t v = x ^ 0x20202020u;
    const uint32_t sg = v & 0x20202020u;
    return v | (sg << 1) | (sg << 2);
}

// Q6_K (210 B, 2-byte aligned): element 128h + 32q + l (l < 32) is
// ql[64h + l + 32(q&1)] (low nibble for q < 2, high for q >= 2) | the
// 2 bits of qh[32h + l] at 2q, minus 32. A unit (h, l0) covers l0..l0+15 of
// all four quarters of half h.
__device__ __forceinline__ void stage_w_q6k(GemmLds &s, const uint8_t *__restrict__ w, int64_t n, int nb,
                                            int64_t r0, int i) {
    for (int idx = threadIdx.x; idx < GM_BN * 5; idx += 256) {
        const int r = idx / 5, u = idx - r * 5;
        const bool ok = r0 + r < n;
        const uint8_t *blk = w + ((r0 + r) * nb + i) * Q6K_BYTES;
        if (u == 4) {
            uint32_t sw[8], d = 0;
#pragma unroll
            for (int j = 0; j < 8; j++) sw[j] = ok ? ld_u16(blk + 192 + 2 * j) : 0u;
            if (ok) d = ld_u16(blk + 208);
#pragma unroll
            for (int j = 0; j < 8; j++) {
                s.sc[r][2 * j] = (int8_t)(sw[j] & 0xffu);
                s.sc[r][2 * j + 1] = (int8_t)(sw[j] >> 8);
            }
            s.wd[r] = h2f(d);
        } else {
            const int h = u >> 1, l0 = 16 * (u & 1);
            uint4 qa = make_uint4(0, 0, 0, 0), qb = qa, qh = qa;
            if (ok) {
                qa = ld16_a2(blk + 64 * h + l0);         // quarters 0 (low) and 2 (high)
                qb = ld16_a2(blk + 64 * h + 32 + l0);    // quarters 1 and 3
                qh = ld16_a2(blk + 128 + 32 * h + l0);
            }
            const uint32_t M = 0x0F0F0F0Fu, T = 0x30303030u;
            const uint32_t a[4] = {qa.x, qa.y, qa.z, qa.w}, b[4] = {qb.x, qb.y, qb.z, qb.w},
                           hh[4] = {qh.x, qh.y, qh.z, qh.w};
            uint32_t o0[4], o1[4], o2[4], o3[4];
#pragma unroll
            for (int k = 0; k < 4; k++) {
                o0[k] = u6_minus_32((a[k] & M) | ((hh[k] << 4) & T));
                o1[k] = u6_minus_32((b[k] & M) | ((hh[k] << 2) & T));
                o2[k] = u6_minus_32(((a[k] >> 4) & M) | (hh[k] & T));
                o3[k] = u6_minus_32(((b[k] >> 4) & M) | ((hh[k] >> 2) & T));
            }
            lds_st16(&s.b[r][128 * h + l0], o0[0], o0[1], o0[2], o0[3]);
            lds_st16(&s.b[r][128 * h + 32 + l0], o1[0], o1[1], o1[2], o1[3]);
            lds_st16(&s.b[r][128 * h + 64 + l0], o2[0], o2[1], o2[2], o2[3]);
            lds_st16(&s.b[r][128 * h + 96 + l0], o3[0], o3[1], o3[2], o3[3]);
        }
    }
}

// Output element v (0..15) of a lane in a 32x32 MFMA tile: column (weight
// row) = lane % 32, row (token) = 8*(v/4) + 4*(lane/32) + v%4.
__device__ __forceinline__ int tok_of(int v, int h) { return 8 * (v >> 2) + 4 * h + (v & 3); }

template <int TYPE, bool FUSED>
__global__ __launch_bounds__(256) void k_gemm(const uint8_t *__restrict__ w, int64_t n, int nb,
                                              const uint8_t *__restrict__ xq, int64_t m, float *__restrict__ y) {
    __shared__ GemmLds s;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int col = lane & 31, h = lane >> 5;
    const int tm = 32 * (wave >> 1), tn = 32 * (wave & 1);   // wave sub-tile in the workgroup tile
    const int64_t r0 = (int64_t)blockIdx.x * GM_BN, t0 = (int64_t)blockIdx.y * GM_BM;
    float sum[16];
#pragma unroll
    for (int v = 0; v < 16; v++) sum[v] = 0.0f;

    for (int i = 0; i < nb; i++) {
        __syncthreads();                                     // previous super-block's reads done
        stage_act(s, xq, m, nb, t0, i);
        if (TYPE == 12) stage_w_q4k(s, w, n, nb, r0, i);
        else if (TYPE == 13) stage_w_q5k(s, w, n, nb, r0, i);
        else stage_w_q6k(s, w, n, nb, r0, i);
        __syncthreads();

        int32_t isum[16];
#pragma unroll
        for (int v = 0; v < 16; v++) isum[v] = 0;
        const int8_t *arow = &s.a[tm + col][0];
        const int8_t *brow = &s.b[tn + col][0];
        const v16i zero = {0};
        if (TYPE == 14) {
#pragma unroll
            for (int sb = 0; sb < 16; sb++) {
                const long av = *(const QK_LDS long *)(arow + 16 * sb + 8 * h);
                const long bv = *(const QK_LDS long *)(brow + 16 * sb + 8 * h);
                const v16i d = __builtin_amdgcn_mfma_i32_32x32x16_i8(av, bv, zero, 0, 0, 0);
                const int32_t scv = s.sc[tn + col][sb];
#pragma unroll
                for (int v = 0; v < 16; v++) isum[v] += __mul24(scv, d[v]);
            }
        } else {
#pragma unroll
            for (int sb = 0; sb < 8; sb++) {
                const v4i av = *(const QK_LDS v4i *)(arow + 32 * sb + 16 * h);
                const v4i bv = *(const QK_LDS v4i *)(brow + 32 * sb + 16 * h);
                const v16i d = __builtin_amdgcn_mfma_i32_32x32x32_i8(av, bv, zero, 0, 0, 0);
                const int32_t scv = s.sc[tn + col][sb];
#pragma unroll
                for (int v = 0; v < 16; v++) isum[v] += __mul24(scv, d[v]);
            }
        }

        const float wd = s.wd[tn + col];
        if (TYPE == 14) {
#pragma unroll
            for (int v = 0; v < 16; v++) {
                const float yd = s.yd[tm + tok_of(v, h)];
                sum[v] = __fadd_rn(sum[v], __fmul_rn(__fmul_rn(wd, yd), (float)isum[v]));
            }
        } else {
            const float wdm = s.wdm[tn + col];
            int32_t mm[8];
#pragma unroll
            for (int j = 0; j < 8; j++) mm[j] = s.mn[tn + col][j];
#pragma unroll
            for (int v = 0; v < 16; v++) {
                const int t = tm + tok_of(v, h);
                const v4i bp = *(const QK_LDS v4i *)&s.bp[t][0];
                int32_t mins = 0;
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    mins += __mul24(mm[2 * q], (int32_t)(int16_t)(bp[q] & 0xffff));
                    mins += __mul24(mm[2 * q + 1], (int32_t)(int16_t)((uint32_t)bp[q] >> 16));
                }
                const float yd = s.yd[t];
                const float d = __fmul_rn(yd, wd);
                const float dmin = __fmul_rn(yd, wdm);
                const float pm = __fmul_rn(dmin, (float)mins);
                const float term = FUSED ? __builtin_fmaf(d, (float)isum[v], -pm)
                                         : __fsub_rn(__fmul_rn(d, (float)isum[v]), pm);
                sum[v] = __fadd_rn(sum[v], term);
            }
        }
    }

    const int64_t row = r0 + tn + col;
    if (row < n) {
#pragma unroll
        for (int v = 0; v < 16; v++) {
            const int64_t t = t0 + tm + tok_of(v, h);
            if (t < m) y[t * n + row] = FUSED ? bcast8(sum[v]) : sum[v];
        }
    }
}

hipError_t launch_gemm(int type, const uint8_t *w, int64_t n, int64_t k, const uint8_t *xq, int64_t m,
                       float *y, int fused, hipStream_t s) {
    const int nb = (int)(k / QK_K);
    const dim3 grid((unsigned)((n + GM_BN - 1) / GM_BN), (unsigned)((m + GM_BM - 1) / GM_BM));
#define QK_GEMM_LAUNCH(T)                                                                            \
    do {                                                                                             \
        if (fused) hipLaunchKernelGGL((k_gemm<T, true>), grid, dim3(256), 0, s, w, n, nb, xq, m, y); \
        else hipLaunchKernelGGL((k_gemm<T, false>), grid, dim3(256), 0, s, w, n, nb, xq, m, y);      \
    } while (0)
    switch (type) {
        case 12: QK_GEMM_LAUNCH(12); break;
        case 13: QK_GEMM_LAUNCH(13); break;
        case 14: QK_GEMM_LAUNCH(14); break;
        default: return hipErrorInvalidValue;
    }
#undef QK_GEMM_LAUNCH
    return hipGetLastError();
}

}  // namespace qk
