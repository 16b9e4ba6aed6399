// qk_chain.hip -- the elementwise links of a decode layer's chain on the
// device (gfx950): residual add + RMSNorm (+ Q8_K of the result), SiLU,
// and SiLU(gate) * up (+ Q8_K), so activations stay in HBM between the
// quantized GEMVs.
//
// Bit-exact restatements of the reference's host code: every float op is
// one IEEE operation with round-to-nearest-even, in the reference's order
// (this file is built with -ffp-contract=off; the only fused multiply-adds
// are the explicit ones inside qk_expf).
#include "qk.h"
#include "qk_dev.h"
#include "qk_expf.h"
#include "qk_kernels.h"

namespace qk {

// v / (1 + expf(-v)): simd_silu_f32's x86 path (simd/simd.c:265-276),
// the same formula as tensor_silu (slm/tensor.c:310-318).
__device__ __forceinline__ float silu(float v) {
    return __fdiv_rn(v, __fadd_rn(1.0f, qk_expf(-v)));
}

// ---- the norm's sequential double sum ----------------------------------
// tensor_rms_norm adds (double)(r_i * r_i) to a double in index order
// (slm/tensor.c:357-360), rounding after every add. The terms are
// non-negative, so while every partial sum of a block of terms (and the
// running sum s before it) is a multiple of 2^g and below 2^(g + 53), no
// add rounds and the block's sequential sum is s + (the exact block sum),
// computed in any order. Each block of NB_T terms therefore gets its sum
// (in a tree), the lowest set bit over its terms and a flag for inf/NaN
// terms in parallel; one lane then walks the blocks in order and adds a
// block in one step when T = s + sum and g = floor(log2 T) + 2 - 53 pass
// the test (T is within a relative 2^-46 of the true total, so the true
// total is below 2^(g + 53) whenever T is below 2^(g + 52)), else adds
// the block's terms one by one as the reference does.
constexpr int NB_T = 64;                               // terms per block (one wave)
constexpr int NB_MAX = QK_NORM_MAX_K / NB_T;

// Exponent of the lowest set bit of a finite double v > 0.
__device__ __forceinline__ int low_bit(double v) {
    const uint64_t b = (uint64_t)__double_as_longlong(v);
    const int e = (int)(b >> 52) & 0x7ff;
    const uint64_t m = (b & 0xfffffffffffffull) | (e ? 0x10000000000000ull : 0);
    return (e ? e : 1) - 1075 + __builtin_ctzll(m);
}

template <int CTRL>
__device__ __forceinline__ double dpp64(double v) {
    const uint64_t b = (uint64_t)__double_as_longlong(v);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_mov_dpp((int)(uint32_t)b, CTRL, 0xF, 0xF, true);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_mov_dpp((int)(uint32_t)(b >> 32), CTRL, 0xF, 0xF, true);
    return __longlong_as_double((long long)(((uint64_t)hi << 32) | lo));
}

__device__ __forceinline__ double readlane64(double v, int l) {
    const uint64_t b = (uint64_t)__double_as_longlong(v);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)b, l);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(b >> 32), l);
    return __longlong_as_double((long long)(((uint64_t)hi << 32) | lo));
}

// Sum over the wave (order irrelevant: used only where it is exact).
__device__ __forceinline__ double wave_sum64(double v) {
    v = __dadd_rn(v, dpp64<0xB1>(v));                 // quad_perm [1,0,3,2]
    v = __dadd_rn(v, dpp64<0x4E>(v));                 // quad_perm [2,3,0,1]
    v = __dadd_rn(v, dpp64<0x141>(v));                // row_half_mirror
    v = __dadd_rn(v, dpp64<0x140>(v));                // row_mirror
    return __dadd_rn(__dadd_rn(readlane64(v, 0), readlane64(v, 16)),
                     __dadd_rn(readlane64(v, 32), readlane64(v, 48)));
}

__device__ __forceinline__ int wave_min_i(int v) {
    v = min(v, __builtin_amdgcn_mov_dpp(v, 0xB1, 0xF, 0xF, true));
    v = min(v, __builtin_amdgcn_mov_dpp(v, 0x4E, 0xF, 0xF, true));
    v = min(v, __builtin_amdgcn_mov_dpp(v, 0x141, 0xF, 0xF, true));
    v = min(v, __builtin_amdgcn_mov_dpp(v, 0x140, 0xF, 0xF, true));
    return min(min(__builtin_amdgcn_readlane(v, 0), __builtin_amdgcn_readlane(v, 16)),
               min(__builtin_amdgcn_readlane(v, 32), __builtin_amdgcn_readlane(v, 48)));
}

// tensor_add (slm/tensor.c:284-291) of an optional delta, then
// tensor_rms_norm (slm/tensor.c:345-367) of the sum, then optionally
// quantize_row_q8_K (slm/tensor.c:683-720) of the normalized row. One
// workgroup of 256 per row of k floats; the row sits in LDS (k * 4 bytes
// of dynamic LDS).
//   r      = h + delta                      (stored to h_out if given)
//   ssq    = sum over i of (double)(r_i * r_i), the sequential double
//            sum in index order (exact blocks in one step, see above)
//   rscale = 1 / sqrtf((float)(ssq / k) + eps)
//   x_i    = (r_i * rscale) * w_i           (stored to x_out if given)
__global__ __launch_bounds__(256) void k_add_rmsnorm(const float *h, const float *__restrict__ delta,
                                                     const float *__restrict__ w, float eps, int64_t k,
                                                     float *h_out, float *__restrict__ x_out,
                                                     uint8_t *__restrict__ xq) {
    extern __shared__ float4 row4[];                   // k / 4 float4
    __shared__ float rscale_s;
    const int64_t t = blockIdx.x;
    const int64_t k4 = k >> 2;
    const float4 *h4 = reinterpret_cast<const float4 *>(h + t * k);
    const float4 *d4 = delta ? reinterpret_cast<const float4 *>(delta + t * k) : nullptr;
    float4 *ho4 = h_out ? reinterpret_cast<float4 *>(h_out + t * k) : nullptr;
    for (int64_t i = threadIdx.x; i < k4; i += 256) {
        float4 v = h4[i];
        if (d4) {
            const float4 a = d4[i];
            v.x = __fadd_rn(v.x, a.x);
            v.y = __fadd_rn(v.y, a.y);
            v.z = __fadd_rn(v.z, a.z);
            v.w = __fadd_rn(v.w, a.w);
        }
        row4[i] = v;
        if (ho4) ho4[i] = v;
    }
    __syncthreads();
    __shared__ double bsum[NB_MAX];
    __shared__ int blow[NB_MAX];                       // lowest set bit; INT_MIN: an inf/NaN term
    const float *rowf = reinterpret_cast<const float *>(row4);
    const int nblk = (int)((k + NB_T - 1) / NB_T);
    {
        const int lane = threadIdx.x & 63;
        for (int b = threadIdx.x >> 6; b < nblk; b += 4) {   // one wave per block
            const int64_t i = (int64_t)b * NB_T + lane;
            const float x = i < k ? rowf[i] : 0.0f;
            const double t = (double)__fmul_rn(x, x);
            const bool special = !(t <= 1.0e308);      // inf or NaN
            const int lb = (t > 0.0 && !special) ? low_bit(t) : 0x7fffffff;
            const double sb = wave_sum64(special ? 0.0 : t);
            const int lbm = wave_min_i(lb);
            const bool any_special = __ballot(special) != 0;   // the whole wave votes
            if (lane == 0) {
                bsum[b] = sb;
                blow[b] = any_special ? (int)0x80000000 : lbm;
            }
        }
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        double ssq = 0.0;
        for (int b = 0; b < nblk; b++) {
            const double T = __dadd_rn(ssq, bsum[b]);
            bool exact = blow[b] != (int)0x80000000;
            if (exact && T > 0.0) {
                const int g = (int)(((uint64_t)__double_as_longlong(T) >> 52) & 0x7ff) - 1023 + 2 - 53;
                exact = blow[b] >= g && (ssq == 0.0 || low_bit(ssq) >= g);
            }
            if (exact) {
                ssq = T;                                // every add of the block was exact
                continue;
            }
            // the block one term at a time: its float4s read first, then
            // the dependent adds (k is a multiple of 4)
            const int64_t q0 = (int64_t)b * (NB_T / 4);
            auto add4 = [&](const float4 v) {
                ssq = __dadd_rn(ssq, (double)__fmul_rn(v.x, v.x));
                ssq = __dadd_rn(ssq, (double)__fmul_rn(v.y, v.y));
                ssq = __dadd_rn(ssq, (double)__fmul_rn(v.z, v.z));
                ssq = __dadd_rn(ssq, (double)__fmul_rn(v.w, v.w));
            };
            if (q0 + NB_T / 4 <= k4) {                  // a whole block
                float4 v[NB_T / 4];
#pragma unroll
                for (int q = 0; q < NB_T / 4; q++) v[q] = row4[q0 + q];
#pragma unroll
                for (int q = 0; q < NB_T / 4; q++) add4(v[q]);
            } else {                                    // the row's last, partial block
                for (int64_t q = q0; q < k4; q++) add4(row4[q]);
            }
        }
        const float ms = __double2float_rn(__ddiv_rn(ssq, (double)k));
        // __builtin_sqrtf is the correctly rounded square root (the raw
        // v_sqrt_f32 that __fsqrt_rn maps to is not)
        rscale_s = __fdiv_rn(1.0f, __builtin_sqrtf(__fadd_rn(ms, eps)));
    }
    __syncthreads();
    const float rscale = rscale_s;
    const float4 *w4 = reinterpret_cast<const float4 *>(w);
    float4 *xo4 = x_out ? reinterpret_cast<float4 *>(x_out + t * k) : nullptr;
    if (xq) {
        // one wave per 256-element block, 4 consecutive elements per lane
        const int lane = threadIdx.x & 63;
        const int64_t nb = k / QK_K;
        for (int64_t b = threadIdx.x >> 6; b < nb; b += 4) {
            const int64_t i = b * 64 + lane;
            const float4 v = row4[i], g = w4[i];
            const float e[4] = {__fmul_rn(__fmul_rn(v.x, rscale), g.x), __fmul_rn(__fmul_rn(v.y, rscale), g.y),
                                __fmul_rn(__fmul_rn(v.z, rscale), g.z), __fmul_rn(__fmul_rn(v.w, rscale), g.w)};
            if (xo4) xo4[i] = make_float4(e[0], e[1], e[2], e[3]);
            uint32_t packed, bs;
            float d;
            q8k_block_wave(e, lane, packed, d, bs);
            uint8_t *out = xq + (t * nb + b) * Q8K_BYTES;
            reinterpret_cast<uint32_t *>(out + 4)[lane] = packed;
            if ((lane & 7) == 0) reinterpret_cast<uint32_t *>(out + 260)[lane >> 3] = bs;
            if (lane == 0) *reinterpret_cast<float *>(out) = d;
        }
    } else {
        for (int64_t i = threadIdx.x; i < k4; i += 256) {
            const float4 v = row4[i], g = w4[i];
            xo4[i] = make_float4(__fmul_rn(__fmul_rn(v.x, rscale), g.x), __fmul_rn(__fmul_rn(v.y, rscale), g.y),
                                 __fmul_rn(__fmul_rn(v.z, rscale), g.z), __fmul_rn(__fmul_rn(v.w, rscale), g.w));
        }
    }
}

// simd_silu_f32 (simd/simd.c:271-277) over n floats; dst may equal src.
__global__ __launch_bounds__(256) void k_silu(const float *src, float *dst, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256)
        dst[i] = silu(src[i]);
}

// The FFN's SwiGLU link: simd_silu_f32 of the gate then tensor_mul
// (slm/tensor.c:293-300) by up (slm/qwen.c:949-954), optionally
// quantized to Q8_K for the down projection. One wave per 256 elements
// of the flattened m x k rows (k a multiple of 256 with xq; of 4
// without), 4 consecutive elements per lane.
__global__ __launch_bounds__(256) void k_swiglu(const float *__restrict__ gate, const float *__restrict__ up,
                                                int64_t n, float *__restrict__ act, uint8_t *__restrict__ xq) {
    const int lane = threadIdx.x & 63;
    const int64_t b = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int64_t i = b * 64 + lane;                   // float4 index
    if (b * QK_K >= n) return;                         // whole wave
    float e[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if (i * 4 < n) {
        const float4 g = reinterpret_cast<const float4 *>(gate)[i];
        const float4 u = reinterpret_cast<const float4 *>(up)[i];
        e[0] = __fmul_rn(silu(g.x), u.x);
        e[1] = __fmul_rn(silu(g.y), u.y);
        e[2] = __fmul_rn(silu(g.z), u.z);
        e[3] = __fmul_rn(silu(g.w), u.w);
        if (act) reinterpret_cast<float4 *>(act)[i] = make_float4(e[0], e[1], e[2], e[3]);
    }
    if (xq) {                                          // n % 256 == 0: every lane is in range
        uint32_t packed, bs;
        float d;
        q8k_block_wave(e, lane, packed, d, bs);
        uint8_t *out = xq + b * Q8K_BYTES;
        reinterpret_cast<uint32_t *>(out + 4)[lane] = packed;
        if ((lane & 7) == 0) reinterpret_cast<uint32_t *>(out + 260)[lane >> 3] = bs;
        if (lane == 0) *reinterpret_cast<float *>(out) = d;
    }
}

// ---- launchers ---------------------------------------------------------
hipError_t launch_add_rmsnorm(const float *h, const float *delta, const float *w, float eps, int64_t m, int64_t k,
                              float *h_out, float *x_out, uint8_t *xq, hipStream_t s) {
    hipLaunchKernelGGL(k_add_rmsnorm, dim3((unsigned)m), dim3(256), (size_t)k * sizeof(float), s, h, delta, w, eps,
                       k, h_out, x_out, xq);
    return hipGetLastError();
}

hipError_t launch_silu(const float *src, float *dst, int64_t n, hipStream_t s) {
    const int64_t want = (n + 255) / 256;
    const unsigned grid = (unsigned)(want < 8192 ? want : 8192);
    hipLaunchKernelGGL(k_silu, dim3(grid), dim3(256), 0, s, src, dst, n);
    return hipGetLastError();
}

hipError_t launch_swiglu(const float *gate, const float *up, int64_t n, float *act, uint8_t *xq, hipStream_t s) {
    const int64_t waves = (n + QK_K - 1) / QK_K;
    hipLaunchKernelGGL(k_swiglu, dim3((unsigned)((waves + 3) / 4)), dim3(256), 0, s, gate, up, n, act, xq);
    return hipGetLastError();
}

}  // namespace qk
