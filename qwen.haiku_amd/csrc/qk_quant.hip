// qk_quant.hip -- activation quantizers and weight dequantizers (gfx950).
//
// Bit-exact restatements of the reference CPU routines: every float op
// is a single IEEE operation with the rounding the reference's x86 build
// performs (no contraction: this file is built with -ffp-contract=off).
#include "qk_dev.h"
#include "qk_kernels.h"

namespace qk {

// quantize_row_q8_K (slm/tensor.c:683-720): one wave per 256-element
// block, 4 elements per lane (q8k_block_wave).
__global__ __launch_bounds__(256) void k_quantize_q8k(const float *__restrict__ x,
                                                      uint8_t *__restrict__ xq,
                                                      int64_t nblocks) {
    const int lane = threadIdx.x & 63;
    const int64_t blk = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (blk >= nblocks) return;                        // whole wave
    const float4 v = reinterpret_cast<const float4 *>(x + blk * QK_K)[lane];
    const float e[4] = {v.x, v.y, v.z, v.w};
    uint32_t packed, bs;
    float d;
    q8k_block_wave(e, lane, packed, d, bs);
    uint8_t *out = xq + blk * Q8K_BYTES;
    reinterpret_cast<uint32_t *>(out + 4)[lane] = packed;
    if ((lane & 7) == 0) reinterpret_cast<uint32_t *>(out + 260)[lane >> 3] = bs;
    if (lane == 0) *reinterpret_cast<float *>(out) = d;
}

// tensor_quantize_row_q8_0 (slm/tensor.c:930-950): 32 lanes per block
// (q80_block_half), d stored as fp16 round-to-nearest-even.
__global__ __launch_bounds__(256) void k_quantize_q8_0(const float *__restrict__ x,
                                                       uint8_t *__restrict__ xq,
                                                       int64_t nblocks) {
    const int lane = threadIdx.x & 31;
    const int64_t blk = ((int64_t)blockIdx.x * 256 + threadIdx.x) >> 5;
    if (blk >= nblocks) return;                        // whole half-wave
    int32_t q;
    float d;
    q80_block_half(x[blk * QK8_0 + lane], q, d);
    uint8_t *out = xq + blk * Q80_BYTES;
    out[2 + lane] = (uint8_t)(q & 0xff);
    if (lane == 0) *reinterpret_cast<uint16_t *>(out) = (uint16_t)f2h(d);
}

// q4k_dequant_block / q5k_dequant_block (slm/tensor.c:800-820, 867-896):
// y = rn(rn(d1*q) - m1), d1 = rn(d*sc), m1 = rn(dmin*m). One thread per
// 4 consecutive outputs of a 64-element chunk.
template <int TYPE>
__global__ __launch_bounds__(256) void k_dequant_q45k(const uint8_t *__restrict__ w,
                                                      float *__restrict__ y, int64_t nblocks) {
    const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t blk = t >> 6;
    if (blk >= nblocks) return;
    const int e0 = (int)(t & 63) * 4;                  // first element, 0..252
    const int c = e0 >> 6, hi = (e0 >> 5) & 1, l0 = e0 & 31;
    const uint8_t *b = w + blk * (TYPE == 12 ? Q4K_BYTES : Q5K_BYTES);
    const uint8_t *qs = b + (TYPE == 12 ? 16 : 48);
    const uint32_t s0 = b[4] | (b[5] << 8) | (b[6] << 16) | ((uint32_t)b[7] << 24);
    const uint32_t s1 = b[8] | (b[9] << 8) | (b[10] << 16) | ((uint32_t)b[11] << 24);
    const uint32_t s2 = b[12] | (b[13] << 8) | (b[14] << 16) | ((uint32_t)b[15] << 24);
    int32_t sc, m;
    scale_min(s0, s1, s2, 2 * c + hi, sc, m);
    const float d1 = __fmul_rn(h2f(ld_u16(b)), (float)sc);
    const float m1 = __fmul_rn(h2f(ld_u16(b + 2)), (float)m);
    float4 o;
    float *op = &o.x;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int l = l0 + i;
        int32_t q = hi ? (qs[32 * c + l] >> 4) : (qs[32 * c + l] & 0x0f);
        if (TYPE == 13) q += ((b[16 + l] >> (2 * c + hi)) & 1) << 4;
        op[i] = __fsub_rn(__fmul_rn(d1, (float)q), m1);
    }
    reinterpret_cast<float4 *>(y + blk * QK_K)[t & 63] = o;
}

// q6k_dequant_block (slm/tensor.c:988-1010): y = rn(rn(d*sc) * (u6-32)).
// Element e: half h = e/128, p = e%128, quarter q = p/32, l = p%32; low
// nibble from ql[64h + l + 32(q&1)] (high nibble when q >= 2), top two
// bits from qh[32h + l] >> 2q.
__global__ __launch_bounds__(256) void k_dequant_q6k(const uint8_t *__restrict__ w,
                                                     float *__restrict__ y, int64_t nblocks) {
    const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t blk = t >> 6;
    if (blk >= nblocks) return;
    const int e0 = (int)(t & 63) * 4;
    const uint8_t *b = w + blk * Q6K_BYTES;
    const float d = h2f(ld_u16(b + 208));
    const float ds = __fmul_rn(d, (float)(int8_t)b[192 + (e0 >> 4)]);
    const int h = e0 >> 7, p = e0 & 127, q = p >> 5, l0 = p & 31;
    float4 o;
    float *op = &o.x;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int l = l0 + i;
        const uint32_t lb = b[64 * h + l + 32 * (q & 1)];
        const int32_t lo = (q >= 2) ? (int32_t)(lb >> 4) : (int32_t)(lb & 0x0f);
        const int32_t hb = (b[128 + 32 * h + l] >> (2 * q)) & 3;
        op[i] = __fmul_rn(ds, (float)((lo | (hb << 4)) - 32));
    }
    reinterpret_cast<float4 *>(y + blk * QK_K)[t & 63] = o;
}

// ---- launchers ---------------------------------------------------------
hipError_t launch_quantize_q8k(const float *x, int64_t nblocks, uint8_t *xq, hipStream_t s) {
    const int64_t grid = (nblocks + 3) / 4;
    hipLaunchKernelGGL(k_quantize_q8k, dim3((unsigned)grid), dim3(256), 0, s, x, xq, nblocks);
    return hipGetLastError();
}

hipError_t launch_quantize_q8_0(const float *x, int64_t nblocks, uint8_t *xq, hipStream_t s) {
    const int64_t grid = (nblocks + 7) / 8;
    hipLaunchKernelGGL(k_quantize_q8_0, dim3((unsigned)grid), dim3(256), 0, s, x, xq, nblocks);
    return hipGetLastError();
}

hipError_t launch_dequant(int type, const uint8_t *w, int64_t nblocks, float *y, hipStream_t s) {
    const int64_t grid = (nblocks * 64 + 255) / 256;
    switch (type) {
        case 12: hipLaunchKernelGGL(k_dequant_q45k<12>, dim3((unsigned)grid), dim3(256), 0, s, w, y, nblocks); break;
        case 13: hipLaunchKernelGGL(k_dequant_q45k<13>, dim3((unsigned)grid), dim3(256), 0, s, w, y, nblocks); break;
        case 14: hipLaunchKernelGGL(k_dequant_q6k, dim3((unsigned)grid), dim3(256), 0, s, w, y, nblocks); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace qk
