// qk_dev.h -- device-side helpers shared by the libqk kernels (gfx950).
//
// Everything here is exact integer work or a single IEEE operation with
// an explicit rounding: the translation units are compiled with
// -ffp-contract=off and each place where the reference's AVX2/VNNI tier
// contracts to an FMA calls __builtin_fmaf by name.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

#define QK_K 256
#define QK8_0 32

// Block byte sizes and field offsets (simd/quants.h:95-130).
#define Q8K_BYTES 292   // f32 d | i8 qs[256] @4 | i16 bsums[16] @260
#define Q4K_BYTES 144   // f16 d | f16 dmin @2 | u8 scales[12] @4 | u8 qs[128] @16
#define Q5K_BYTES 176   // ... scales @4 | u8 qh[32] @16 | u8 qs[128] @48
#define Q6K_BYTES 210   // u8 ql[128] | u8 qh[64] @128 | i8 scales[16] @192 | f16 d @208
#define Q80_BYTES 34    // f16 d | i8 qs[32] @2


namespace qk {

// ---- fp16 <-> fp32 (the reference's `_Float16` casts on x86: exact
// widening, round-to-nearest-even narrowing; narrowing is integer work so
// it does not depend on the MODE register).
__device__ __forceinline__ float h2f(uint32_t h) {
    // v_cvt_f32_f16: exact widening; fp16 denormals are kept (the kernels
    // run with denorm mode 3 for f16/f64).
    return __half2float(__ushort_as_half((unsigned short)(h & 0xffffu)));
}

__device__ __forceinline__ uint32_t f2h(float f) {
    uint32_t x = __float_as_uint(f);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7fffffffu;
    uint32_t q;
    if (ax > 0x7f800000u) {
        q = 0x7e00u | ((ax >> 13) & 0x3ffu);
    } else if (ax >= 0x477ff000u) {
        q = 0x7c00u;
    } else if (ax >= 0x38800000u) {
        uint32_t rem = ax & 0x1fffu;
        q = (((ax >> 23) - 112u) << 10) | ((ax >> 13) & 0x3ffu);
        if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) q += 1;
    } else if (ax <= 0x33000000u) {
        q = 0;
    } else {
        uint32_t m = (ax & 0x7fffffu) | 0x800000u;
        uint32_t shift = 126u - (ax >> 23);
        uint32_t rem = m & ((1u << shift) - 1u), half = 1u << (shift - 1);
        q = m >> shift;
        if (rem > half || (rem == half && (q & 1u))) q += 1;
    }
    return sign | q;
}

// q_nearest_int (simd/quants.h:137-142): magic-number rounding with a
// separately rounded add.
__device__ __forceinline__ int32_t nearest_int(float v) {
    float t = __fadd_rn(v, 12582912.f);
    return (__float_as_int(t) & 0x007fffff) - 0x00400000;
}

// ---- 4-wide int8 dot (v_dot4_i32_i8): exact int32 accumulate.
__device__ __forceinline__ int32_t dot4(uint32_t a, uint32_t b, int32_t c) {
    return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
}

// ---- cross-lane helpers within aligned groups of 8 lanes -------------
__device__ __forceinline__ int32_t dpp_xor1(int32_t v) {
    return __builtin_amdgcn_mov_dpp(v, 0xB1, 0xF, 0xF, true);   // quad_perm [1,0,3,2]
}
__device__ __forceinline__ int32_t dpp_xor2(int32_t v) {
    return __builtin_amdgcn_mov_dpp(v, 0x4E, 0xF, 0xF, true);   // quad_perm [2,3,0,1]
}
__device__ __forceinline__ int32_t dpp_hmirror(int32_t v) {
    return __builtin_amdgcn_mov_dpp(v, 0x141, 0xF, 0xF, true);  // row_half_mirror
}
// Sum over the 8-lane group; every lane of the group gets the total.
__device__ __forceinline__ int32_t sum8(int32_t v) {
    v += dpp_xor1(v);
    v += dpp_xor2(v);
    v += dpp_hmirror(v);
    return v;
}
// Lane l <- lane l^4 (ds_swizzle bit mode, xor_mask 4, within 32 lanes).
__device__ __forceinline__ float swz_xor4(float v) {
    return __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x101F));
}
__device__ __forceinline__ float swz_xor1(float v) {
    return __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x041F));
}
__device__ __forceinline__ float swz_xor2(float v) {
    return __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x081F));
}

// ---- loads -------------------------------------------------------------
// Weight and activation pointers reach the kernels inside argument structs,
// where the compiler only sees generic pointers; the casts below make
// every such load a global_load (not flat_load).
#if defined(__HIP_DEVICE_COMPILE__)
#define QK_GLOBAL __attribute__((address_space(1)))
#define QK_LDS __attribute__((address_space(3)))
#else
#define QK_GLOBAL   /* host pass: device bodies are parsed, never run */
#define QK_LDS
#endif

__device__ __forceinline__ uint4 ld16(const uint8_t *p) {       // 16-B aligned
    return *(const QK_GLOBAL uint4 *)(p);
}

__device__ __forceinline__ uint32_t ld32(const uint8_t *p) {    // 4-B aligned
    return *(const QK_GLOBAL uint32_t *)(p);
}

__device__ __forceinline__ uint32_t ld_u16(const uint8_t *p) {  // 2-B aligned
    return *(const QK_GLOBAL uint16_t *)(p);
}

__device__ __forceinline__ uint32_t ld_u8(const uint8_t *p) {
    return *(const QK_GLOBAL uint8_t *)(p);
}

// Buffer loads: offsets past the resource's byte range read zeros without
// a memory access, so a load needs no per-lane guard.
__device__ __forceinline__ uint32_t bl32(__amdgpu_buffer_rsrc_t r, int off) {
    return __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0);
}
__device__ __forceinline__ uint4 bl128(__amdgpu_buffer_rsrc_t r, int off) {    // 4-byte aligned offset
    const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
    return make_uint4(v[0], v[1], v[2], v[3]);
}

// ---- Q4_K / Q5_K 6-bit scale and min of sub-block s (0..7) from the
// 12 packed bytes held in three dwords (q4k_get_scale_min,
// simd/quants.h:215-224).
__device__ __forceinline__ uint32_t sbyte(uint32_t s0, uint32_t s1, uint32_t s2, int i) {
    uint32_t d = (i < 4) ? s0 : ((i < 8) ? s1 : s2);
    return (d >> (8 * (i & 3))) & 0xffu;
}
__device__ __forceinline__ void scale_min(uint32_t s0, uint32_t s1, uint32_t s2, int s,
                                          int32_t &sc, int32_t &m) {
    if (s < 4) {
        sc = (int32_t)(sbyte(s0, s1, s2, s) & 63u);
        m  = (int32_t)(sbyte(s0, s1, s2, s + 4) & 63u);
    } else {
        sc = (int32_t)((sbyte(s0, s1, s2, s + 4) & 15u) | ((sbyte(s0, s1, s2, s - 4) >> 6) << 4));
        m  = (int32_t)((sbyte(s0, s1, s2, s + 4) >> 4) | ((sbyte(s0, s1, s2, s) >> 6) << 4));
    }
}

// ---- activation block quantizers (one wave / half-wave per block) --------
// Both restate the reference bit for bit; the callers store the results
// where their layout wants them (global Q8_K / Q8_0 rows, or an LDS copy
// of a row inside a GEMV workgroup).

// Largest value over the wave (inputs NaN-free): DPP within each 16-lane
// row, then the four row results read as uniform values.
__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, __int_as_float(dpp_xor1(__float_as_int(v))));
    v = fmaxf(v, __int_as_float(dpp_xor2(__float_as_int(v))));
    v = fmaxf(v, __int_as_float(dpp_hmirror(__float_as_int(v))));
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x140, 0xF, 0xF, true)));  // row_mirror
    const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
    const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
    const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
    const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
    return fmaxf(fmaxf(r0, r1), fmaxf(r2, r3));
}

// One Q8_K block (quantize_row_q8_K, slm/tensor.c:683-720) by one wave,
// elements 4 lane .. 4 lane + 3 in e[]. Results: `packed` = this lane's
// four quants as bytes; `d` (wave-uniform); `bs` = bsums 2p | 2p+1 << 16
// for lanes 8p (other lanes: don't care).
//  * amax/xmax: the first element with the largest |x| (strict '>' in a
//    sequential scan; NaN never compares greater, so it is never chosen).
//    The wave takes the largest |x| (NaN as 0), then the first lane
//    holding it (ballot) supplies its first such element.
//  * iscale = -127/xmax, d = 1/iscale (IEEE division),
//    q = clamp(nearest_int(iscale*x)), bsums over 16-element groups.
__device__ __forceinline__ void q8k_block_wave(const float (&e)[4], int lane, uint32_t &packed, float &d,
                                               uint32_t &bs) {
    float a[4], la = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float ax = fabsf(e[i]);
        a[i] = (ax != ax) ? 0.0f : ax;
        la = fmaxf(la, a[i]);
    }
    const float amax = wave_max(la);
    // this lane's first element at amax (scanning backwards keeps the first)
    float mine = e[3];
#pragma unroll
    for (int i = 2; i >= 0; i--) mine = a[i] == amax ? e[i] : mine;
    const uint64_t hit = __ballot(la == amax);
    const int first = __builtin_ctzll(hit);            // amax == 0: lane 0, unused
    const float xmax = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(mine), first));
    int32_t q[4] = {0, 0, 0, 0};
    d = 0.0f;
    if (amax != 0.0f) {
        const float iscale = __fdiv_rn(-127.0f, xmax);
        d = __fdiv_rn(1.0f, iscale);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            int32_t t = nearest_int(__fmul_rn(iscale, e[i]));
            q[i] = t > 127 ? 127 : (t < -128 ? -128 : t);
        }
    }
    packed = (uint32_t)(q[0] & 0xff) | ((uint32_t)(q[1] & 0xff) << 8) | ((uint32_t)(q[2] & 0xff) << 16) |
             ((uint32_t)(q[3] & 0xff) << 24);
    // bsums[j] = sum of lanes 4j..4j+3; lane 8p gets bsums 2p, 2p+1 (lane
    // 8p+4's sum arrives by DPP row_shl:4, inside the 16-lane row)
    int32_t sm = q[0] + q[1] + q[2] + q[3];
    sm += dpp_xor1(sm);
    sm += dpp_xor2(sm);
    const int32_t s_next = __builtin_amdgcn_mov_dpp(sm, 0x104, 0xF, 0xF, true);
    bs = ((uint32_t)sm & 0xffffu) | ((uint32_t)s_next << 16);
}

// One Q8_0 block (tensor_quantize_row_q8_0, slm/tensor.c:930-950) by 32
// lanes (lanes 0-31 and 32-63 of a wave take one block each): this lane's
// quant and the block's d (before its fp16 store). d = amax/127,
// id = 1/d (of the unrounded d), q = (int)roundf(x*id) (half away from
// zero).
__device__ __forceinline__ void q80_block_half(float v, int32_t &q, float &d) {
    float a = fabsf(v);
    a = (a != a) ? 0.0f : a;                           // '>' never picks NaN
    // block maximum: DPP within each 16-lane row, then the two rows of
    // this half-wave's block (read as uniform values)
    a = fmaxf(a, __int_as_float(dpp_xor1(__float_as_int(a))));
    a = fmaxf(a, __int_as_float(dpp_xor2(__float_as_int(a))));
    a = fmaxf(a, __int_as_float(dpp_hmirror(__float_as_int(a))));
    a = fmaxf(a, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(a), 0x140, 0xF, 0xF, true)));
    const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(a), 0));
    const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(a), 16));
    const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(a), 32));
    const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(a), 48));
    a = (threadIdx.x & 32) ? fmaxf(r2, r3) : fmaxf(r0, r1);
    d = __fdiv_rn(a, 127.0f);
    const float id = (d != 0.0f) ? __fdiv_rn(1.0f, d) : 0.0f;
    // Saturating conversion, as the reference's clang build behaves when
    // d underflows and id = 1/d is inf.
    const float r = roundf(__fmul_rn(v, id));
    q = r >= 127.0f ? 127 : (r <= -128.0f ? -128 : (int32_t)r);
}

// ---- float epilogues (bit-exact per tier) --------------------------------
// Q4_K/Q5_K super-block term. separate (scalar/AVX1, simd/quants.h:305,
// simd/avx.c:654): rn(rn(d*isum) - rn(dmin*mins)); fused (AVX2/VNNI,
// simd/avx.c:229,466,515): fma(d, isum, -rn(dmin*mins)).
template <bool FUSED>
__device__ __forceinline__ float kterm(float yd, uint32_t xd, uint32_t xdmin, int32_t isum,
                                       int32_t mins) {
    float d = __fmul_rn(yd, h2f(xd));
    float dmin = __fmul_rn(yd, h2f(xdmin));
    float pm = __fmul_rn(dmin, (float)mins);
    float t;
    if (FUSED) {
        t = __builtin_fmaf(d, (float)isum, -pm);
    } else {
        t = __fsub_rn(__fmul_rn(d, (float)isum), pm);
    }
    return t;
}

// AVX2/VNNI return the row sum through an 8-lane broadcast:
// hsum(8 x s) / 8 (simd/avx.c:231-240), which is s unless 8s overflows.
// The three doublings of the sum are exact unless they overflow, and so
// is s * 8, at the same exponent: both give 8s or the same infinity.
__device__ __forceinline__ float bcast8(float s) {
    return __fmul_rn(__fmul_rn(s, 8.0f), 0.125f);   // x / 8 and x * 2^-3 round the same exact value
}

// Stores outputs v0 .. v0 + NV - 1 of one lane of a 32x32 MFMA tile
// (v_mfma_i32_32x32x*: output v of lane l is token 8(v / 4) + 4(l / 32) +
// v % 4 of the tile and weight row l % 32) as y[t * n + row], where the
// tile's tokens start at t0 + tm; outputs whose tile token is mrows or
// more (past the tokens this tile holds) are not stored. One lane pointer, stepped by n to the
// next token or by 5n past the fourth of a group of four, so no 64-bit
// product per output.
template <bool FUSED, int NV>
__device__ __forceinline__ void store_mfma32(float *__restrict__ y, int64_t n, int64_t row, int64_t t0, int tm,
                                             int mrows, int v0, int h, const float *s) {
    const int tb = tm + 8 * (v0 >> 2) + 4 * h + (v0 & 3);
    float *yp = y + (uint64_t)(uint32_t)(t0 + tb) * (uint64_t)n + row;
#pragma unroll
    for (int i = 0; i < NV; i++) {
        const int v = v0 + i;
        if (tm + 8 * (v >> 2) + 4 * h + (v & 3) < mrows)
            __builtin_nontemporal_store(FUSED ? bcast8(s[i]) : s[i], yp);
        yp += (v & 3) == 3 ? 5 * n : n;
    }
}

// Q6_K term (all tiers, simd/quants.h:399): rn(rn(fp16(x.d)*y.d) * (float)v).
__device__ __forceinline__ float q6term(float yd, uint32_t xd, int32_t v) {
    return __fmul_rn(__fmul_rn(h2f(xd), yd), (float)v);
}

}  // namespace qk
