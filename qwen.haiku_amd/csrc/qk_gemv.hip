// qk_gemv.hip -- decode GEMV over native GGUF blocks (gfx950).
//
// One kernel serves every decode matmul: a launch carries up to 16
// descriptors (type, W, xq, y), so a layer's projections go out as one
// dispatch. A 256-thread workgroup computes row tiles of one descriptor
// (grid-stride over tiles).
//
// Each workgroup streams tiles of consecutive rows (one contiguous byte
// range) from HBM into LDS with fully coalesced 16-byte loads, double
// buffered, and computes from LDS: an aligned group of 4 lanes owns one
// 256-element super-block, each lane takes 32 quant bytes and runs
// v_dot4 against the activation bytes; the group sums its int32 partials
// with DPP. Super-block terms of a row are then added in block order by
// one lane, so the float sum rounds exactly as the reference's sequential
// `sum += term` (simd/quants.h:305, simd/avx.c:467).
//
// Activations are staged once per workgroup into LDS with 16-byte
// aligned quant rows (Q8_K: qs[nb][256] | bsums[nb][16] | d[nb]).
#include "qk_dev.h"
#include "qk_kernels.h"

namespace qk {

// ---- activation staging ----------------------------------------------------
__device__ __forceinline__ void stage_q8k(const uint8_t *__restrict__ xq, int nb, uint8_t *lds) {
    uint32_t *qs = reinterpret_cast<uint32_t *>(lds);
    uint32_t *bs = reinterpret_cast<uint32_t *>(lds + nb * 256);
    float *d = reinterpret_cast<float *>(lds + nb * 288);
    for (int i = threadIdx.x; i < nb * 73; i += blockDim.x) {
        const int b = i / 73, r = i - b * 73;
        const uint32_t v = ld32(xq + 4 * i);
        if (r == 0) d[b] = __uint_as_float(v);
        else if (r <= 64) qs[b * 64 + r - 1] = v;
        else bs[b * 8 + r - 65] = v;
    }
}

// Q8_0 activation row: qs[nb][32] | d[nb] (fp16 widened once).
__device__ __forceinline__ void stage_q80(const uint8_t *__restrict__ xq, int nb, uint8_t *lds) {
    uint16_t *qs = reinterpret_cast<uint16_t *>(lds);
    float *d = reinterpret_cast<float *>(lds + nb * 32);
    for (int i = threadIdx.x; i < nb * 17; i += blockDim.x) {
        const int b = i / 17, r = i - b * 17;
        const uint32_t v = ld_u16(xq + 2 * i);
        if (r == 0) d[b] = h2f(v);
        else qs[b * 16 + r - 1] = (uint16_t)v;
    }
}

#define M4 0x0F0F0F0Fu

__device__ __forceinline__ int32_t dot16(uint32_t w0, uint32_t w1, uint32_t w2, uint32_t w3,
                                         const uint4 a) {
    int32_t s = dot4(w0, a.x, 0);
    s = dot4(w1, a.y, s);
    s = dot4(w2, a.z, s);
    return dot4(w3, a.w, s);
}

// ---- LDS reads (activation row) ------------------------------------------------
__device__ __forceinline__ uint4 lds16(const uint8_t *p) {          // 16-B aligned
    return *(const QK_LDS uint4 *)(p);
}
__device__ __forceinline__ uint32_t lds32(const uint8_t *p) {       // 4-B aligned
    return *(const QK_LDS uint32_t *)(p);
}

__device__ __forceinline__ int32_t sum4(int32_t v) {
    v += dpp_xor1(v);
    v += dpp_xor2(v);
    return v;
}

__device__ __forceinline__ int32_t dot32(const uint32_t (&w)[8], const uint8_t *a) {
    const uint4 a0 = lds16(a), a1 = lds16(a + 16);
    int32_t s = dot4(w[0], a0.x, 0);
    s = dot4(w[1], a0.y, s);
    s = dot4(w[2], a0.z, s);
    s = dot4(w[3], a0.w, s);
    s = dot4(w[4], a1.x, s);
    s = dot4(w[5], a1.y, s);
    s = dot4(w[6], a1.z, s);
    return dot4(w[7], a1.w, s);
}

__device__ __forceinline__ int32_t bsum_pair(const uint8_t *act, int nb, int b, int s) {
    const uint32_t v = lds32(act + nb * 256 + b * 32 + 4 * s);
    return (int32_t)(int16_t)(v & 0xffffu) + (int32_t)(int16_t)(v >> 16);
}

// ---- per-super-block raw loads and terms ------------------------------------
// A group of 4 lanes owns one 256-element super-block; lane j (0..3)
// loads 32 quant bytes of it straight from HBM into registers. Loads are
// split from the arithmetic so the next work item's bytes are in flight
// while the current one is reduced.
template <int T> struct Raw;
template <> struct Raw<12> { uint4 hdr, q0, q1; };
template <> struct Raw<13> { uint4 hdr, q0, q1, h0, h1; };
template <> struct Raw<14> { uint32_t l[9], h[9], sh, sc, sc2, d; };

// Q4_K (simd/quants.h:267-306): lane j holds chunk c = j, qs[32j..32j+32):
// low nibbles pair with q8[64j..64j+32) under scale 2j, high nibbles with
// q8[64j+32..64j+64) under scale 2j+1; mins 2j, 2j+1 meet bsum pairs 2j,
// 2j+1.
__device__ __forceinline__ void load_sb(Raw<12> &r, const uint8_t *__restrict__ blk, int j) {
    r.hdr = ld16(blk);
    r.q0 = ld16(blk + 16 + 32 * j);
    r.q1 = ld16(blk + 32 + 32 * j);
}

template <bool FUSED>
__device__ __forceinline__ float term_sb(const Raw<12> &r, int b, int j, const uint8_t *act, int nb) {
    const uint32_t q[8] = {r.q0.x, r.q0.y, r.q0.z, r.q0.w, r.q1.x, r.q1.y, r.q1.z, r.q1.w};
    uint32_t lo[8], hi[8];
#pragma unroll
    for (int i = 0; i < 8; i++) {
        lo[i] = q[i] & M4;
        hi[i] = (q[i] >> 4) & M4;
    }
    const uint8_t *a = act + b * 256 + 64 * j;
    const int32_t slo = dot32(lo, a), shi = dot32(hi, a + 32);
    int32_t sc0, m0, sc1, m1;
    scale_min(r.hdr.y, r.hdr.z, r.hdr.w, 2 * j, sc0, m0);
    scale_min(r.hdr.y, r.hdr.z, r.hdr.w, 2 * j + 1, sc1, m1);
    const int32_t isum = sum4(slo * sc0 + shi * sc1);
    const int32_t mins = sum4(m0 * bsum_pair(act, nb, b, 2 * j) + m1 * bsum_pair(act, nb, b, 2 * j + 1));
    const float yd = ((const QK_LDS float *)(act + nb * 288))[b];
    return kterm<FUSED>(yd, r.hdr.x & 0xffffu, r.hdr.x >> 16, isum, mins);
}

// Q5_K (simd/quants.h:310-351): as Q4_K plus bit 2j / 2j+1 of qh[l].
__device__ __forceinline__ void load_sb(Raw<13> &r, const uint8_t *__restrict__ blk, int j) {
    r.hdr = ld16(blk);
    r.h0 = ld16(blk + 16);
    r.h1 = ld16(blk + 32);
    r.q0 = ld16(blk + 48 + 32 * j);
    r.q1 = ld16(blk + 64 + 32 * j);
}

template <bool FUSED>
__device__ __forceinline__ float term_sb(const Raw<13> &r, int b, int j, const uint8_t *act, int nb) {
    const uint32_t q[8] = {r.q0.x, r.q0.y, r.q0.z, r.q0.w, r.q1.x, r.q1.y, r.q1.z, r.q1.w};
    const uint32_t qh[8] = {r.h0.x, r.h0.y, r.h0.z, r.h0.w, r.h1.x, r.h1.y, r.h1.z, r.h1.w};
    const uint32_t s0 = 2 * j, s1 = 2 * j + 1;
    uint32_t lo[8], hi[8];
#pragma unroll
    for (int i = 0; i < 8; i++) {
        lo[i] = (q[i] & M4) | (((qh[i] >> s0) & 0x01010101u) << 4);
        hi[i] = ((q[i] >> 4) & M4) | (((qh[i] >> s1) & 0x01010101u) << 4);
    }
    const uint8_t *a = act + b * 256 + 64 * j;
    const int32_t slo = dot32(lo, a), shi = dot32(hi, a + 32);
    int32_t sc0, m0, sc1, m1;
    scale_min(r.hdr.y, r.hdr.z, r.hdr.w, 2 * j, sc0, m0);
    scale_min(r.hdr.y, r.hdr.z, r.hdr.w, 2 * j + 1, sc1, m1);
    const int32_t isum = sum4(slo * sc0 + shi * sc1);
    const int32_t mins = sum4(m0 * bsum_pair(act, nb, b, 2 * j) + m1 * bsum_pair(act, nb, b, 2 * j + 1));
    const float yd = ((const QK_LDS float *)(act + nb * 288))[b];
    return kterm<FUSED>(yd, r.hdr.x & 0xffffu, r.hdr.x >> 16, isum, mins);
}

// Q6_K (simd/quants.h:356-402). Lane j = 2h + qq holds ql bytes
// [32j, 32j+32) (positions l = 0..31 of half h, quarter qq): the low
// nibble is element 128h + 32qq + l, the high nibble element +64; the two
// top bits come from qh[32h + l] bits 2qq and 2qq+4. Sub-blocks
// 8h+2qq+{0,1} (low) and +4 (high). Each lane folds its share of
// isum - 32*isum_mins, exact in int32, so one reduction suffices. 210-byte
// blocks are 2-byte aligned: 32-byte runs are read as aligned 36-byte
// windows (inside the block: the last ends at byte 196) and funnel-shifted.
__device__ __forceinline__ void load_sb(Raw<14> &r, const uint8_t *__restrict__ blk, int j) {
    const int h = j >> 1, qq = j & 1;
    const uint32_t sh = (uint32_t)reinterpret_cast<uintptr_t>(blk) & 3u;
    r.sh = sh;
    const uint8_t *wl = blk + 32 * j - sh;
    const uint8_t *wh = blk + 128 + 32 * h - sh;
    const u32x4a4 l0 = ld16_a4(wl), l1 = ld16_a4(wl + 16);
    const u32x4a4 h0 = ld16_a4(wh), h1 = ld16_a4(wh + 16);
    r.l[0] = l0.x; r.l[1] = l0.y; r.l[2] = l0.z; r.l[3] = l0.w;
    r.l[4] = l1.x; r.l[5] = l1.y; r.l[6] = l1.z; r.l[7] = l1.w; r.l[8] = ld32(wl + 32);
    r.h[0] = h0.x; r.h[1] = h0.y; r.h[2] = h0.z; r.h[3] = h0.w;
    r.h[4] = h1.x; r.h[5] = h1.y; r.h[6] = h1.z; r.h[7] = h1.w; r.h[8] = ld32(wh + 32);
    const int s = 8 * h + 2 * qq;
    r.sc = ld_u16(blk + 192 + s);
    r.sc2 = ld_u16(blk + 196 + s);
    r.d = ld_u16(blk + 208);
}

template <bool FUSED>
__device__ __forceinline__ float term_sb(const Raw<14> &r, int b, int j, const uint8_t *act, int nb) {
    const int h = j >> 1, qq = j & 1;
    const uint32_t sh = r.sh, sa = 2 * qq;
    uint32_t lo[8], hi[8];
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const uint32_t ql = __builtin_amdgcn_alignbyte(r.l[i + 1], r.l[i], sh);
        const uint32_t qh = __builtin_amdgcn_alignbyte(r.h[i + 1], r.h[i], sh) >> sa;
        lo[i] = (ql & M4) | ((qh << 4) & 0x30303030u);
        hi[i] = ((ql >> 4) & M4) | (qh & 0x30303030u);
    }
    const int s = 8 * h + 2 * qq;                      // sub-blocks s, s+1 | s+4, s+5
    const uint8_t *a = act + b * 256 + 16 * s;
    const int32_t d0 = dot16(lo[0], lo[1], lo[2], lo[3], lds16(a));
    const int32_t d1 = dot16(lo[4], lo[5], lo[6], lo[7], lds16(a + 16));
    const int32_t d4 = dot16(hi[0], hi[1], hi[2], hi[3], lds16(a + 64));
    const int32_t d5 = dot16(hi[4], hi[5], hi[6], hi[7], lds16(a + 80));
    const int32_t sc0 = (int32_t)(int8_t)(r.sc & 0xffu), sc1 = (int32_t)(int8_t)(r.sc >> 8);
    const int32_t sc4 = (int32_t)(int8_t)(r.sc2 & 0xffu), sc5 = (int32_t)(int8_t)(r.sc2 >> 8);
    const uint32_t bl = lds32(act + nb * 256 + b * 32 + 2 * s);
    const uint32_t bh = lds32(act + nb * 256 + b * 32 + 2 * s + 8);
    const int32_t b0 = (int16_t)(bl & 0xffffu), b1 = (int16_t)(bl >> 16);
    const int32_t b4 = (int16_t)(bh & 0xffffu), b5 = (int16_t)(bh >> 16);
    const int32_t v = d0 * sc0 + d1 * sc1 + d4 * sc4 + d5 * sc5 - 32 * (b0 * sc0 + b1 * sc1 + b4 * sc4 + b5 * sc5);
    const int32_t tot = sum4(v);
    const float yd = ((const QK_LDS float *)(act + nb * 288))[b];
    return q6term(yd, r.d, tot);
}

// Monotone 64-bit key: larger logit first, lower index on ties; -0 == +0
// and NaN below everything (sample_argmax never picks a NaN).
__device__ __forceinline__ uint64_t argkey(float v, int64_t row) {
    uint32_t b = __float_as_uint(v);
    if (v == 0.0f) b = 0;
    uint32_t key = (v != v) ? 0u : ((b & 0x80000000u) ? ~b : (b | 0x80000000u));
    return ((uint64_t)key << 32) | (uint64_t)(0xffffffffu - (uint32_t)row);
}

// Rows of one K-quant descriptor handled by this workgroup: tiles
// lw, lw+nwg, ... of 4 waves x 16/P rows. A row's P groups each take every
// P-th super-block; the P terms of a step are gathered with ds_bpermute
// and added to the row sum in super-block order. Work items (tile, step)
// are pipelined one deep: item i+1's loads are issued before item i is
// reduced. The activation row is staged after the first loads are out.
template <int TYPE, bool FUSED>
__device__ __forceinline__ void run_kq(const GemvDesc &D, int lw, int nwg, uint8_t *lds, uint64_t &best) {
    constexpr int BB = TYPE == 12 ? Q4K_BYTES : (TYPE == 13 ? Q5K_BYTES : Q6K_BYTES);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int grp = lane >> 2, j = lane & 3;
    const int lp = 31 - __builtin_clz(D.p);
    const int P = 1 << lp;
    const int team = grp >> lp, g = grp & (P - 1);
    const int nb = D.nb, rpt = D.rows_per_tile, ntiles = D.ntiles;
    const int niter = (nb + P - 1) >> lp;
    const int64_t n = D.n;
    const uint8_t *__restrict__ w = D.w;
    float *__restrict__ y = D.y;
    const int src0 = team * P * 4;
    const int64_t rofs = (int64_t)wave * (16 >> lp) + team;
    auto issue = [&](Raw<TYPE> &r, int t, int i) {
        const int64_t row = (int64_t)t * rpt + rofs;
        const int b = i * P + g;
        if (t < ntiles && row < n && b < nb) load_sb(r, w + (row * nb + b) * BB, j);
    };
    int tile = lw, it = 0;
    Raw<TYPE> cur;
    issue(cur, tile, it);
    stage_q8k(D.xq, nb, lds);
    __syncthreads();
    float sum = 0.0f;
    while (tile < ntiles) {
        int ntile = tile, nit = it + 1;
        if (nit == niter) { nit = 0; ntile += nwg; }
        Raw<TYPE> nxt;
        issue(nxt, ntile, nit);
        const int64_t row = (int64_t)tile * rpt + rofs;
        const int b = it * P + g;
        float t = 0.0f;
        if (row < n && b < nb) t = term_sb<FUSED>(cur, b, j, lds, nb);
        const int lim = (nb - it * P < P) ? nb - it * P : P;
        for (int g2 = 0; g2 < lim; g2++) sum += __shfl(t, src0 + 4 * g2);
        if (it == niter - 1) {
            if (FUSED) sum = bcast8(sum);
            if (row < n && g == 0 && j == 0) {
                *(QK_GLOBAL float *)(y + row) = sum;
                const uint64_t k = argkey(sum, row);
                best = k > best ? k : best;
            }
            sum = 0.0f;
        }
        cur = nxt;
        tile = ntile;
        it = nit;
    }
}

// Q8_0 (q8_0_dot_q8_0, simd/avx.c:65-158, simd/quants.h:244-256): one row
// per wave. Lane = slot s (bytes 4s..4s+3 of a block, the AVX lane) +
// 8 x phase; phases take blocks b = phase + 8i, so a chunk of 64 blocks
// is loaded by the whole wave at once. The per-block slot partials p and
// scales go through LDS to 8 chain lanes, which run the reference's
// sequential accumulation over blocks:
//  fused (AVX2/VNNI): acc_s = fma((float)p_s, s_b, acc_s), then
//        ((a0+a4)+(a1+a5)) + ((a2+a6)+(a3+a7));
//  separate (scalar/AVX1): sum = sum + (float)(sum_s p_s) * s_b.
template <bool FUSED>
__device__ __forceinline__ void run_q80(const GemvDesc &D, int lw, int nwg, uint8_t *lds, uint64_t &best) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int s = lane & 7, ph = lane >> 3;
    const int nb = D.nb, ntiles = D.ntiles;
    const int64_t n = D.n;
    const uint8_t *__restrict__ w = D.w;
    float *__restrict__ y = D.y;
    stage_q80(D.xq, nb, lds);
    __syncthreads();
    const QK_LDS uint32_t *aq = (const QK_LDS uint32_t *)(lds);
    const QK_LDS float *ad = (const QK_LDS float *)(lds + nb * 32);
    // per-wave exchange area after the staged activations: 8 slots x 64
    // blocks of partials (slot-major, so a chain lane reads contiguous
    // 16-byte vectors) and 64 block scales
    QK_LDS int32_t *xp = (QK_LDS int32_t *)(lds + D.lds_act + wave * 64 * 36);
    QK_LDS float *xs = (QK_LDS float *)(xp + 64 * 8);
    for (int tile = lw; tile < ntiles; tile += nwg) {
        const int64_t row = (int64_t)tile * 4 + wave;
        if (row >= n) continue;                        // wave-uniform
        const uint8_t *rowp = w + row * (int64_t)nb * Q80_BYTES;
        float acc = 0.0f;
        for (int c0 = 0; c0 < nb; c0 += 64) {
            const int cn = (nb - c0 < 64) ? nb - c0 : 64;
            uint32_t wq[8], wd[8];
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const int b = c0 + ph + 8 * i;
                if (ph + 8 * i < cn) {
                    const uint8_t *blk = rowp + (int64_t)b * Q80_BYTES;
                    wq[i] = ld_u16(blk + 2 + 4 * s) | (ld_u16(blk + 4 + 4 * s) << 16);
                    wd[i] = ld_u16(blk);
                }
            }
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const int bl = ph + 8 * i;
                if (bl < cn) {
                    const int b = c0 + bl;
                    const int32_t p = dot4(wq[i], aq[b * 8 + s], 0);
                    const float sc = __fmul_rn(h2f(wd[i]), ad[b]);
                    if (FUSED) {
                        xp[s * 64 + bl] = p;
                        if (s == 0) xs[bl] = sc;
                    } else {
                        const int32_t sumi = sum8(p);
                        if (s == 0) xs[bl] = __fmul_rn((float)sumi, sc);
                    }
                }
            }
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            if (ph == 0) {
                int bl = 0;
                if (FUSED) {
                    for (; bl + 4 <= cn; bl += 4) {
                        const int4 pv = *(const QK_LDS int4 *)(xp + s * 64 + bl);
                        const float4 sv = *(const QK_LDS float4 *)(xs + bl);
                        acc = __builtin_fmaf((float)pv.x, sv.x, acc);
                        acc = __builtin_fmaf((float)pv.y, sv.y, acc);
                        acc = __builtin_fmaf((float)pv.z, sv.z, acc);
                        acc = __builtin_fmaf((float)pv.w, sv.w, acc);
                    }
                    for (; bl < cn; bl++) acc = __builtin_fmaf((float)xp[s * 64 + bl], xs[bl], acc);
                } else {
                    for (; bl + 4 <= cn; bl += 4) {
                        const float4 sv = *(const QK_LDS float4 *)(xs + bl);
                        acc = __fadd_rn(acc, sv.x);
                        acc = __fadd_rn(acc, sv.y);
                        acc = __fadd_rn(acc, sv.z);
                        acc = __fadd_rn(acc, sv.w);
                    }
                    for (; bl < cn; bl++) acc = __fadd_rn(acc, xs[bl]);
                }
            }
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        }
        float r = acc;
        if (FUSED) {
            r = __fadd_rn(r, swz_xor4(r));
            r = __fadd_rn(r, swz_xor1(r));
            r = __fadd_rn(r, swz_xor2(r));
        }
        if (lane == 0) {
            *(QK_GLOBAL float *)(y + row) = r;
            const uint64_t k = argkey(r, row);
            best = k > best ? k : best;
        }
    }
}

// One launch, up to 16 descriptors. Workgroups [wg0, wg0 + nwg) of a
// launch belong to descriptor d.
template <bool FUSED>
__global__ __launch_bounds__(256, 6) void k_gemv(GemvArgs args, uint64_t *__restrict__ amax_partial,
                                              uint32_t *__restrict__ zero_ctr) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    if (zero_ctr && blockIdx.x == 0 && threadIdx.x == 0) *zero_ctr = 0;   // top-k candidate counter
    int di = 0;
    while (di + 1 < args.count && (int)blockIdx.x >= args.d[di + 1].wg0) di++;
    const GemvDesc &D = args.d[di];
    const int lw = (int)blockIdx.x - D.wg0;
    uint64_t best = 0;
    switch (D.type) {
        case 12: run_kq<12, FUSED>(D, lw, D.nwg, lds, best); break;
        case 13: run_kq<13, FUSED>(D, lw, D.nwg, lds, best); break;
        case 14: run_kq<14, FUSED>(D, lw, D.nwg, lds, best); break;
        default: run_q80<FUSED>(D, lw, D.nwg, lds, best); break;
    }
    if (amax_partial) {
        // Workgroup maximum of the argmax keys of every row it wrote.
        __shared__ uint64_t wbest[4];
        uint64_t v = best;
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) {
            const uint32_t lo = __shfl_xor((uint32_t)v, off);
            const uint32_t hi = __shfl_xor((uint32_t)(v >> 32), off);
            const uint64_t o = ((uint64_t)hi << 32) | lo;
            v = o > v ? o : v;
        }
        if ((threadIdx.x & 63) == 0) wbest[threadIdx.x >> 6] = v;
        __syncthreads();
        if (threadIdx.x == 0) {
            uint64_t m = wbest[0];
            for (int i = 1; i < 4; i++) m = wbest[i] > m ? wbest[i] : m;
            amax_partial[blockIdx.x] = m;
        }
    }
}

void gemv_plan(GemvDesc &d) {
    if (d.type == 8) {
        d.nb = (int32_t)(d.k / QK8_0);
        d.p = 1;
        d.rows_per_tile = 4;
        d.lds_act = (d.nb * 36 + 15) & ~15;
    } else {
        d.nb = (int32_t)(d.k / QK_K);
        // groups per row: enough to cover the row in one step up to 16
        // super-blocks (k <= 4096), so a row costs one memory latency
        int p = 1;
        while (p < 16 && p < d.nb) p *= 2;
        d.p = p;
        d.rows_per_tile = 4 * (16 / p);
        d.lds_act = (d.nb * 292 + 15) & ~15;
    }
    d.tr = d.rows_per_tile;
    d.tile_cap = 0;
    d.ntiles = (int32_t)((d.n + d.rows_per_tile - 1) / d.rows_per_tile);
    d.nwg = d.ntiles;
}

// Rows are not staged, so any row length up to the activation limit works.
int64_t gemv_max_row_bytes() { return (int64_t)1 << 40; }

static hipError_t launch_gemv_impl(GemvArgs &a, int max_wg_per_desc, uint64_t *amax_partial,
                                   uint32_t *zero_ctr, int *grid_out, hipStream_t s) {
    // Workgroups dispatch in blockIdx order. The longest-latency
    // descriptors (Q8_0's per-row FMA chain, then the widest rows) take
    // the first workgroups, so they start first.
    auto rank = [](const GemvDesc &d) { return d.type == 8 ? 0 : (int)(64 - d.nb); };
    for (int i = 1; i < a.count; i++) {
        GemvDesc t = a.d[i];
        int k = i - 1;
        while (k >= 0 && rank(a.d[k]) > rank(t)) { a.d[k + 1] = a.d[k]; k--; }
        a.d[k + 1] = t;
    }
    int32_t wg = 0, lds = 0;
    for (int i = 0; i < a.count; i++) {
        GemvDesc &d = a.d[i];
        d.nwg = d.ntiles < max_wg_per_desc ? d.ntiles : max_wg_per_desc;
        d.wg0 = wg;
        wg += d.nwg;
        const int32_t need = d.lds_act + (d.type == 8 ? 4 * 64 * 36 : 0);
        lds = need > lds ? need : lds;
    }
    a.lds_bytes = lds;
    if (grid_out) *grid_out = wg;
    if (a.fused)
        hipLaunchKernelGGL(k_gemv<true>, dim3(wg), dim3(256), lds, s, a, amax_partial, zero_ctr);
    else
        hipLaunchKernelGGL(k_gemv<false>, dim3(wg), dim3(256), lds, s, a, amax_partial, zero_ctr);
    return hipGetLastError();
}

hipError_t launch_gemv(GemvArgs &a, int max_grid, hipStream_t s) {
    return launch_gemv_impl(a, max_grid, nullptr, nullptr, nullptr, s);
}

// ---- LM head: exact argmax and top-k -------------------------------------
// The GEMV leaves one key per workgroup: the maximum (value, -row) key of
// the rows it wrote. argmax = max over those keys.
//
// Top-k (keys compare by value, then lower row): the k-th largest of the
// workgroup maxima is a lower bound T on the k-th largest logit (the k
// largest maxima are k distinct logits >= T), so every top-k logit has a
// value key >= T. k_topk_filter finds T (radix select over the maxima)
// and collects the logits >= T; k_topk_final ranks those candidates (by
// counting when they fit one block, else after a radix select of the k
// best). If more than TOPK_CAND logits pass the filter (a pathological
// flat distribution), k_topk_final falls back to k exact passes over all
// logits.
#define TOPK_CAND 4096
#define LMHEAD_MAX_WG 4096                             // argmax partials (one per workgroup)
#define LMHEAD_WG 1024                                 // workgroups of the LM-head GEMV (grid-stride
                                                       // over tiles): fewer maxima for the top-k bound

__device__ __forceinline__ uint32_t valkey(float v) {
    uint32_t b = __float_as_uint(v);
    if (v == 0.0f) b = 0;
    return (v != v) ? 0u : ((b & 0x80000000u) ? ~b : (b | 0x80000000u));
}

// Exact k-th largest of the keys held by a 1024-thread block (R keys per
// thread, `have` masks the valid ones), 8 bits per pass from the top, NB
// bits in total. hist: 256 + 2 words of LDS.
template <int R, int NB, typename K>
__device__ K block_kth_largest(const K (&key)[R], const bool (&have)[R], int k, uint32_t *hist) {
    K prefix = 0, mask = 0;
    int need = k;
    const int lane = threadIdx.x & 63;
    uint32_t *sel = hist + 256;                        // [0] digit, [1] keys above it
    for (int shift = NB - 8; shift >= 0; shift -= 8) {
        if (threadIdx.x < 256) hist[threadIdx.x] = 0;
        __syncthreads();
#pragma unroll
        for (int r = 0; r < R; r++)
            if (have[r] && (key[r] & mask) == prefix) atomicAdd(&hist[(uint32_t)(key[r] >> shift) & 255u], 1u);
        __syncthreads();
        if (threadIdx.x < 64) {
            // lane l owns digits 255-4l .. 252-4l (descending); suffix scan
            uint32_t c[4], tot = 0;
#pragma unroll
            for (int q = 0; q < 4; q++) { c[q] = hist[255 - 4 * lane - q]; tot += c[q]; }
            uint32_t incl = tot;
#pragma unroll
            for (int off = 1; off < 64; off <<= 1) {
                const uint32_t o = __shfl_up(incl, off);
                if (lane >= off) incl += o;
            }
            const uint32_t excl = incl - tot;
            if (excl < (uint32_t)need && incl >= (uint32_t)need) {
                uint32_t above = excl;
                int q = 0;
                while (above + c[q] < (uint32_t)need) { above += c[q]; q++; }
                sel[0] = 255 - 4 * lane - q;
                sel[1] = above;
            }
        }
        __syncthreads();
        prefix |= (K)sel[0] << shift;
        mask |= (K)255 << shift;
        need -= (int)sel[1];
        __syncthreads();
    }
    return prefix;
}

// Grid: ceil(n / 4096) blocks of 1024. Every block finds the same T from
// the nparts (<= LMHEAD_MAX_WG) workgroup maxima, then filters its 4096
// logits.
__global__ __launch_bounds__(1024) void k_topk_filter(const float *__restrict__ logits, int64_t n,
                                                      const uint64_t *__restrict__ partial, int nparts,
                                                      int topk, uint64_t *__restrict__ cand,
                                                      uint32_t *__restrict__ ctr) {
    __shared__ uint32_t hist[258];
    uint32_t key[4];
    bool have[4];
#pragma unroll
    for (int r = 0; r < 4; r++) {
        const int i = threadIdx.x + 1024 * r;
        have[r] = i < nparts;
        key[r] = have[r] ? (uint32_t)(partial[i] >> 32) : 0u;
    }
    const int64_t base = (int64_t)blockIdx.x * 4096;
    float v[4];
#pragma unroll
    for (int r = 0; r < 4; r++) {
        const int64_t i = base + threadIdx.x + 1024 * r;
        v[r] = i < n ? logits[i] : 0.0f;
    }
    // Fewer maxima than k (a tiny vocabulary): no bound, every logit passes.
    const uint32_t T = (nparts >= topk) ? block_kth_largest<4, 32, uint32_t>(key, have, topk, hist) : 0u;
#pragma unroll
    for (int r = 0; r < 4; r++) {
        const int64_t i = base + threadIdx.x + 1024 * r;
        if (i < n && valkey(v[r]) >= T) {
            const uint32_t slot = atomicAdd(ctr, 1u);
            if (slot < TOPK_CAND) cand[slot] = ((uint64_t)valkey(v[r]) << 32) | (0xffffffffu - (uint32_t)i);
        }
    }
}

// One block of 1024: argmax from the per-workgroup maxima; the exact top-k
// of the filtered candidates, ranked value-descending / row-ascending.
__global__ __launch_bounds__(1024) void k_topk_final(const float *__restrict__ logits, int64_t n,
                                                     const uint64_t *__restrict__ partial, int nparts,
                                                     const uint64_t *__restrict__ cand,
                                                     const uint32_t *__restrict__ ctr, int topk,
                                                     int32_t *__restrict__ argmax,
                                                     int32_t *__restrict__ topk_idx,
                                                     float *__restrict__ topk_val) {
    __shared__ uint32_t hist[258];
    __shared__ uint64_t win[1024];                     // candidates (ranking) or winners
    __shared__ uint64_t red[16];
    __shared__ uint32_t nwin;
    // argmax: max of the partial keys
    uint64_t m = 0;
    for (int i = threadIdx.x; i < nparts; i += 1024) m = partial[i] > m ? partial[i] : m;
    const uint32_t c = topk > 0 ? *ctr : 0u;
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const uint32_t lo = __shfl_xor((uint32_t)m, off), hi = __shfl_xor((uint32_t)(m >> 32), off);
        const uint64_t o = ((uint64_t)hi << 32) | lo;
        m = o > m ? o : m;
    }
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
    if (threadIdx.x == 0) nwin = 0;
    __syncthreads();
    if (threadIdx.x == 0) {
        uint64_t b = red[0];
        for (int i = 1; i < 16; i++) b = red[i] > b ? red[i] : b;
        int32_t best = (int32_t)(0xffffffffu - (uint32_t)(b & 0xffffffffu));
        const float l0 = logits[0];
        if (l0 != l0) best = 0;                        // sample_argmax: v[0] = NaN never loses
        *argmax = best;
    }
    if (topk <= 0) return;                             // uniform
    int nw;                                            // keys in win[] to rank
    if (c <= 1024) {
        // Few candidates: rank every one of them directly.
        if (threadIdx.x < c) win[threadIdx.x] = cand[threadIdx.x];
        nw = (int)c;
    } else if (c <= TOPK_CAND) {
        uint64_t key[4];
        bool have[4];
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const uint32_t i = threadIdx.x + 1024 * r;
            have[r] = i < c;
            key[r] = have[r] ? cand[i] : 0;
        }
        const uint64_t T = block_kth_largest<4, 64, uint64_t>(key, have, topk, hist);
#pragma unroll
        for (int r = 0; r < 4; r++)
            if (have[r] && key[r] >= T) win[atomicAdd(&nwin, 1u)] = key[r];
        nw = topk;
    } else {
        // Fallback: k exact passes, each taking the largest key below the
        // previous winner.
        uint64_t prev = ~(uint64_t)0;
        for (int r = 0; r < topk; r++) {
            uint64_t b = 0;
            for (int64_t i = threadIdx.x; i < n; i += 1024) {
                const uint64_t kk = ((uint64_t)valkey(logits[i]) << 32) | (0xffffffffu - (uint32_t)i);
                if (kk < prev && kk > b) b = kk;
            }
#pragma unroll
            for (int off = 32; off > 0; off >>= 1) {
                const uint32_t lo = __shfl_xor((uint32_t)b, off), hi = __shfl_xor((uint32_t)(b >> 32), off);
                const uint64_t o = ((uint64_t)hi << 32) | lo;
                b = o > b ? o : b;
            }
            __syncthreads();
            if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = b;
            __syncthreads();
            uint64_t bb = red[0];
            for (int i = 1; i < 16; i++) bb = red[i] > bb ? red[i] : bb;
            if (threadIdx.x == 0) win[r] = bb;
            prev = bb;
        }
        nw = topk;
    }
    __syncthreads();
    // Rank the keys (all distinct) and write the topk best in order.
    if ((int)threadIdx.x < nw) {
        const uint64_t me = win[threadIdx.x];
        int rank = 0;
        for (int i = 0; i < nw; i++) rank += win[i] > me;
        if (rank < topk) {
            const int32_t idx = (int32_t)(0xffffffffu - (uint32_t)(me & 0xffffffffu));
            topk_idx[rank] = idx;
            topk_val[rank] = logits[idx];
        }
    }
}

static int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

size_t lmhead_cand_bytes(int64_t, int) {
    // argmax partials (<= 4096 workgroups) | candidate keys | counter
    return (size_t)(LMHEAD_MAX_WG + TOPK_CAND) * sizeof(uint64_t) + 64;
}

hipError_t launch_lmhead(const uint8_t *w, int64_t n, int64_t k, const uint8_t *xq, int topk,
                         float *logits, int32_t *argmax, int32_t *topk_idx, float *topk_val,
                         void *scratch, int fused, hipStream_t s) {
    GemvArgs a{};
    a.count = 1;
    a.fused = fused;
    a.d[0].type = 14;
    a.d[0].n = n;
    a.d[0].k = k;
    a.d[0].w = w;
    a.d[0].xq = xq;
    a.d[0].y = logits;
    gemv_plan(a.d[0]);
    uint64_t *partial = reinterpret_cast<uint64_t *>(scratch);
    uint64_t *cand = partial + LMHEAD_MAX_WG;
    uint32_t *ctr = reinterpret_cast<uint32_t *>(cand + TOPK_CAND);
    int grid = 0;
    hipError_t e = launch_gemv_impl(a, LMHEAD_WG, partial, ctr, &grid, s);
    if (e != hipSuccess) return e;
    if (grid > LMHEAD_MAX_WG) return hipErrorInvalidValue;
    if (topk > 0) {
        hipLaunchKernelGGL(k_topk_filter, dim3((unsigned)cdiv(n, 4096)), dim3(1024), 0, s, logits, n, partial,
                           grid, topk, cand, ctr);
        if ((e = hipGetLastError()) != hipSuccess) return e;
    }
    hipLaunchKernelGGL(k_topk_final, dim3(1), dim3(1024), 0, s, logits, n, partial, grid, cand, ctr, topk,
                       argmax, topk_idx, topk_val);
    return hipGetLastError();
}

}  // namespace qk
