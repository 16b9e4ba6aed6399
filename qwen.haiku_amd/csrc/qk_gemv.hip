// qk_gemv.hip -- decode GEMV over native GGUF blocks (gfx950).
//
// One kernel serves every decode matmul: a launch carries up to 16
// descriptors (type, W, xq, y), so a layer's projections go out as one
// dispatch. A 256-thread workgroup computes one row tile of one
// descriptor at a time (grid-stride over tiles).
//
// Lane mapping for the K-quants: an aligned group of 8 lanes owns one
// 256-element super-block; each lane streams 16 contiguous quant bytes
// of it (128-bit loads; the 8 lanes of a group read 128 contiguous
// bytes), takes its 16+16 activation bytes from LDS, and runs v_dot4.
// The group then sums its int32 partials with DPP. P groups (1,2,4,8)
// cooperate on one row, each taking every P-th super-block; the P terms
// of a step are gathered with ds_bpermute and added to the row sum in
// super-block order, so the float sum rounds exactly as the reference's
// sequential `sum += term` (simd/quants.h:305, simd/avx.c:467).
//
// Activations are staged once per workgroup into LDS with 16-byte
// aligned quant rows (Q8_K: qs[nb][256] | bsums[nb][16] | d[nb]).
#include "qk_dev.h"
#include "qk_kernels.h"

namespace qk {

// ---- activation staging ----------------------------------------------------
__device__ __forceinline__ void stage_q8k(const uint8_t *__restrict__ xq, int nb, uint8_t *lds) {
    const uint32_t *src = reinterpret_cast<const uint32_t *>(xq);
    uint32_t *qs = reinterpret_cast<uint32_t *>(lds);
    uint32_t *bs = reinterpret_cast<uint32_t *>(lds + nb * 256);
    float *d = reinterpret_cast<float *>(lds + nb * 288);
    for (int i = threadIdx.x; i < nb * 73; i += blockDim.x) {
        const int b = i / 73, r = i - b * 73;
        const uint32_t v = src[i];
        if (r == 0) d[b] = __uint_as_float(v);
        else if (r <= 64) qs[b * 64 + r - 1] = v;
        else bs[b * 8 + r - 65] = v;
    }
}

// Q8_0 activation row: qs[nb][32] | d[nb] (fp16 widened once).
__device__ __forceinline__ void stage_q80(const uint8_t *__restrict__ xq, int nb, uint8_t *lds) {
    const uint16_t *src = reinterpret_cast<const uint16_t *>(xq);
    uint16_t *qs = reinterpret_cast<uint16_t *>(lds);
    float *d = reinterpret_cast<float *>(lds + nb * 32);
    for (int i = threadIdx.x; i < nb * 17; i += blockDim.x) {
        const int b = i / 17, r = i - b * 17;
        const uint32_t v = src[i];
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

// ---- per-super-block terms (called by all 8 lanes of a group) -------------
// Q4_K (simd/quants.h:267-306): lane j holds qs[16j..16j+16) = chunk
// c = j/2, positions l = 16(j&1)..+16: low nibbles pair with q8[64c+l]
// under scale 2c, high nibbles with q8[64c+32+l] under scale 2c+1. Lane
// j also contributes min j times bsum pair j.
template <bool FUSED>
__device__ __forceinline__ float term_q4k(const uint8_t *__restrict__ blk, int b, int j,
                                          const uint8_t *lds, int nb) {
    const uint4 hdr = ld16(blk);
    const uint4 q = ld16(blk + 16 + 16 * j);
    const int c = j >> 1, h = j & 1;
    const uint8_t *a = lds + b * 256;
    const uint4 alo = *reinterpret_cast<const uint4 *>(a + 64 * c + 16 * h);
    const uint4 ahi = *reinterpret_cast<const uint4 *>(a + 64 * c + 32 + 16 * h);
    const int32_t slo = dot16(q.x & M4, q.y & M4, q.z & M4, q.w & M4, alo);
    const int32_t shi = dot16((q.x >> 4) & M4, (q.y >> 4) & M4, (q.z >> 4) & M4, (q.w >> 4) & M4, ahi);
    int32_t sc0, m0, sc1, m1, scj, mj;
    scale_min(hdr.y, hdr.z, hdr.w, 2 * c, sc0, m0);
    scale_min(hdr.y, hdr.z, hdr.w, 2 * c + 1, sc1, m1);
    scale_min(hdr.y, hdr.z, hdr.w, j, scj, mj);
    const uint32_t bsp = reinterpret_cast<const uint32_t *>(lds + nb * 256 + b * 32)[j];
    const int32_t pair = (int32_t)(int16_t)(bsp & 0xffffu) + (int32_t)(int16_t)(bsp >> 16);
    const int32_t isum = sum8(slo * sc0 + shi * sc1);
    const int32_t mins = sum8(mj * pair);
    const float yd = reinterpret_cast<const float *>(lds + nb * 288)[b];
    return kterm<FUSED>(yd, hdr.x & 0xffffu, hdr.x >> 16, isum, mins);
}

// Q5_K (simd/quants.h:310-351): as Q4_K plus bit 2c / 2c+1 of qh[l].
template <bool FUSED>
__device__ __forceinline__ float term_q5k(const uint8_t *__restrict__ blk, int b, int j,
                                          const uint8_t *lds, int nb) {
    const uint4 hdr = ld16(blk);
    const int c = j >> 1, h = j & 1;
    const uint4 qh = ld16(blk + 16 + 16 * h);
    const uint4 q = ld16(blk + 48 + 16 * j);
    const uint8_t *a = lds + b * 256;
    const uint4 alo = *reinterpret_cast<const uint4 *>(a + 64 * c + 16 * h);
    const uint4 ahi = *reinterpret_cast<const uint4 *>(a + 64 * c + 32 + 16 * h);
    const uint32_t s0 = 2 * c, s1 = 2 * c + 1;
#define Q5LO(qv, hv) (((qv) & M4) | ((((hv) >> s0) & 0x01010101u) << 4))
#define Q5HI(qv, hv) ((((qv) >> 4) & M4) | ((((hv) >> s1) & 0x01010101u) << 4))
    const int32_t slo = dot16(Q5LO(q.x, qh.x), Q5LO(q.y, qh.y), Q5LO(q.z, qh.z), Q5LO(q.w, qh.w), alo);
    const int32_t shi = dot16(Q5HI(q.x, qh.x), Q5HI(q.y, qh.y), Q5HI(q.z, qh.z), Q5HI(q.w, qh.w), ahi);
#undef Q5LO
#undef Q5HI
    int32_t sc0, m0, sc1, m1, scj, mj;
    scale_min(hdr.y, hdr.z, hdr.w, 2 * c, sc0, m0);
    scale_min(hdr.y, hdr.z, hdr.w, 2 * c + 1, sc1, m1);
    scale_min(hdr.y, hdr.z, hdr.w, j, scj, mj);
    const uint32_t bsp = reinterpret_cast<const uint32_t *>(lds + nb * 256 + b * 32)[j];
    const int32_t pair = (int32_t)(int16_t)(bsp & 0xffffu) + (int32_t)(int16_t)(bsp >> 16);
    const int32_t isum = sum8(slo * sc0 + shi * sc1);
    const int32_t mins = sum8(mj * pair);
    const float yd = reinterpret_cast<const float *>(lds + nb * 288)[b];
    return kterm<FUSED>(yd, hdr.x & 0xffffu, hdr.x >> 16, isum, mins);
}

// Q6_K (simd/quants.h:356-402). Lane j = 4h + 2qq + lh holds ql bytes
// [16j, 16j+16): element 128h + 32qq + 16lh + i takes the low nibble,
// element +64 the high nibble; the two high bits come from
// qh[32h + 16lh + i] bits 2qq and 2qq+4. Sub-blocks s = 8h+2qq+lh and
// s+4. Each lane folds its share of isum - 32*isum_mins, which is exact
// in int32, so one reduction suffices. Blocks are 2-byte aligned (210 B),
// so the quant bytes are read through aligned 20-byte windows that stay
// inside the block.
__device__ __forceinline__ float term_q6k(const uint8_t *__restrict__ blk, int b, int j,
                                          const uint8_t *lds, int nb) {
    const int h = j >> 2, qq = (j >> 1) & 1, lh = j & 1;
    const uint4 ql = ld16_a2(blk + 16 * j);
    const uint4 qh = ld16_a2(blk + 128 + 32 * h + 16 * lh);
    const int slo = 8 * h + 2 * qq + lh, shi = slo + 4;
    const uint32_t sa = 2 * qq, sb = 2 * qq + 4;
#define Q6LO(lv, hv) (((lv) & M4) | ((((hv) >> sa) & 0x03030303u) << 4))
#define Q6HI(lv, hv) ((((lv) >> 4) & M4) | ((((hv) >> sb) & 0x03030303u) << 4))
    const uint8_t *a = lds + b * 256;
    const uint4 alo = *reinterpret_cast<const uint4 *>(a + 16 * slo);
    const uint4 ahi = *reinterpret_cast<const uint4 *>(a + 16 * shi);
    const int32_t dl = dot16(Q6LO(ql.x, qh.x), Q6LO(ql.y, qh.y), Q6LO(ql.z, qh.z), Q6LO(ql.w, qh.w), alo);
    const int32_t dh = dot16(Q6HI(ql.x, qh.x), Q6HI(ql.y, qh.y), Q6HI(ql.z, qh.z), Q6HI(ql.w, qh.w), ahi);
#undef Q6LO
#undef Q6HI
    const int32_t sclo = (int8_t)blk[192 + slo], schi = (int8_t)blk[192 + shi];
    const int16_t *bs = reinterpret_cast<const int16_t *>(lds + nb * 256 + b * 32);
    const int32_t v = dl * sclo + dh * schi - 32 * ((int32_t)bs[slo] * sclo + (int32_t)bs[shi] * schi);
    const int32_t tot = sum8(v);
    const float yd = reinterpret_cast<const float *>(lds + nb * 288)[b];
    return q6term(yd, ld_u16(blk + 208), tot);
}

// Monotone 64-bit key: larger logit first, lower index on ties; -0 == +0
// and NaN below everything (sample_argmax never picks a NaN).
__device__ __forceinline__ uint64_t argkey(float v, int64_t row) {
    uint32_t b = __float_as_uint(v);
    if (v == 0.0f) b = 0;
    uint32_t key = (v != v) ? 0u : ((b & 0x80000000u) ? ~b : (b | 0x80000000u));
    return ((uint64_t)key << 32) | (uint64_t)(0xffffffffu - (uint32_t)row);
}

// Row tile of a K-quant matrix: 4 waves x (8/P) rows.
template <int TYPE, bool FUSED>
__device__ __forceinline__ void tile_kq(const uint8_t *__restrict__ w, int64_t n, int nb, int lp,
                                        int rows_per_tile, int64_t rt, const uint8_t *lds,
                                        float *__restrict__ y, uint64_t &best) {
    constexpr int BB = TYPE == 12 ? Q4K_BYTES : (TYPE == 13 ? Q5K_BYTES : Q6K_BYTES);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int grp = lane >> 3, j = lane & 7;
    const int P = 1 << lp;
    const int team = grp >> lp, g = grp & (P - 1);
    const int64_t row = rt * rows_per_tile + wave * (8 >> lp) + team;
    const bool active = row < n;
    const uint8_t *rowp = w + (active ? row : 0) * (int64_t)nb * BB;
    const int src0 = team * P * 8;
    float sum = 0.0f;
    for (int i = 0; i < nb; i += P) {
        const int b = i + g;
        float t = 0.0f;
        if (active && b < nb) {
            if (TYPE == 12) t = term_q4k<FUSED>(rowp + (int64_t)b * BB, b, j, lds, nb);
            else if (TYPE == 13) t = term_q5k<FUSED>(rowp + (int64_t)b * BB, b, j, lds, nb);
            else t = term_q6k(rowp + (int64_t)b * BB, b, j, lds, nb);
        }
        const int lim = (nb - i < P) ? nb - i : P;
        for (int g2 = 0; g2 < lim; g2++) sum += __shfl(t, src0 + 8 * g2);
    }
    if (FUSED) sum = bcast8(sum);
    if (active && g == 0 && j == 0) {
        y[row] = sum;
        const uint64_t k = argkey(sum, row);
        best = k > best ? k : best;
    }
}

// Q8_0 row tile: 8 lanes per row (lane j = the reference's AVX lane j:
// bytes 4j..4j+3 of every block), 32 rows per tile.
//  fused (AVX2/VNNI, simd/avx.c:65-123): acc_j = fma((float)p_j, s_b, acc_j)
//        over blocks, then ((a0+a4)+(a1+a5)) + ((a2+a6)+(a3+a7));
//  separate (scalar/AVX1, simd/quants.h:244-256): sum += (float)sumi * s_b.
template <bool FUSED>
__device__ __forceinline__ void tile_q80(const uint8_t *__restrict__ w, int64_t n, int nb,
                                         int64_t rt, const uint8_t *lds, float *__restrict__ y,
                                         uint64_t &best) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int grp = lane >> 3, j = lane & 7;
    const int64_t row = rt * 32 + wave * 8 + grp;
    if (row >= n) return;                              // whole 8-lane group
    const uint8_t *rowp = w + row * (int64_t)nb * Q80_BYTES;
    const uint32_t *aq = reinterpret_cast<const uint32_t *>(lds);
    const float *ad = reinterpret_cast<const float *>(lds + nb * 32);
    float acc = 0.0f;
#pragma unroll 4
    for (int b = 0; b < nb; b++) {
        const uint8_t *blk = rowp + (int64_t)b * Q80_BYTES;
        const uint32_t wq = ld_u16(blk + 2 + 4 * j) | (ld_u16(blk + 4 + 4 * j) << 16);
        const int32_t p = dot4(wq, aq[b * 8 + j], 0);
        const float s = __fmul_rn(h2f(ld_u16(blk)), ad[b]);
        if (FUSED) {
            acc = __builtin_fmaf((float)p, s, acc);
        } else {
            const int32_t sumi = sum8(p);
            acc = __fadd_rn(acc, __fmul_rn((float)sumi, s));
        }
    }
    float r = acc;
    if (FUSED) {
        r = __fadd_rn(r, swz_xor4(r));
        r = __fadd_rn(r, swz_xor1(r));
        r = __fadd_rn(r, swz_xor2(r));
    }
    if (j == 0) {
        y[row] = r;
        const uint64_t k = argkey(r, row);
        best = k > best ? k : best;
    }
}

template <bool FUSED>
__global__ __launch_bounds__(256) void k_gemv(GemvArgs args, uint64_t *__restrict__ amax_partial) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    const GemvArgs *A = &args;
    const int count = A->count, tiles_total = A->tiles_total;
    int cur = -1;
    uint64_t best = 0;
    for (int tile = blockIdx.x; tile < tiles_total; tile += gridDim.x) {
        int di = 0;
        while (di + 1 < count && tile >= A->d[di + 1].tile0) di++;
        const int32_t type = A->d[di].type;
        const int32_t nb = A->d[di].nb;
        const uint8_t *xq = A->d[di].xq;
        if (di != cur) {
            if (cur >= 0) __syncthreads();
            if (type == 8) stage_q80(xq, nb, lds);
            else stage_q8k(xq, nb, lds);
            __syncthreads();
            cur = di;
        }
        const uint8_t *w = A->d[di].w;
        const int64_t n = A->d[di].n;
        float *y = A->d[di].y;
        const int lp = A->d[di].p == 8 ? 3 : (A->d[di].p == 4 ? 2 : (A->d[di].p == 2 ? 1 : 0));
        const int rpt = A->d[di].rows_per_tile;
        const int64_t rt = tile - A->d[di].tile0;
        switch (type) {
            case 12: tile_kq<12, FUSED>(w, n, nb, lp, rpt, rt, lds, y, best); break;
            case 13: tile_kq<13, FUSED>(w, n, nb, lp, rpt, rt, lds, y, best); break;
            case 14: tile_kq<14, FUSED>(w, n, nb, lp, rpt, rt, lds, y, best); break;
            default: tile_q80<FUSED>(w, n, nb, rt, lds, y, best); break;
        }
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
        __syncthreads();
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
        d.rows_per_tile = 32;
    } else {
        d.nb = (int32_t)(d.k / QK_K);
        int p = 1;
        while (p < 8 && 2 * p <= d.nb) p *= 2;
        d.p = p;
        d.rows_per_tile = 4 * (8 / p);
    }
    d.ntiles = (int32_t)((d.n + d.rows_per_tile - 1) / d.rows_per_tile);
}

static hipError_t launch_gemv_impl(GemvArgs &a, int max_grid, uint64_t *amax_partial,
                                   int *grid_out, hipStream_t s) {
    int32_t t = 0, lds = 0;
    for (int i = 0; i < a.count; i++) {
        a.d[i].tile0 = t;
        t += a.d[i].ntiles;
        const int32_t need = a.d[i].type == 8 ? a.d[i].nb * 36 : a.d[i].nb * 292;
        lds = need > lds ? need : lds;
    }
    a.tiles_total = t;
    a.lds_bytes = (lds + 15) & ~15;
    int grid = t < max_grid ? t : max_grid;
    if (grid < 1) grid = 1;
    if (grid_out) *grid_out = grid;
    if (a.fused)
        hipLaunchKernelGGL(k_gemv<true>, dim3(grid), dim3(256), a.lds_bytes, s, a, amax_partial);
    else
        hipLaunchKernelGGL(k_gemv<false>, dim3(grid), dim3(256), a.lds_bytes, s, a, amax_partial);
    return hipGetLastError();
}

hipError_t launch_gemv(GemvArgs &a, int max_grid, hipStream_t s) {
    return launch_gemv_impl(a, max_grid, nullptr, nullptr, s);
}

// ---- LM head: argmax finalize and exact top-k -------------------------------
#define TOPK_SORT 4096

// Bitonic sort (descending) of TOPK_SORT keys in LDS by 1024 threads.
__device__ void bitonic_desc(uint64_t *k) {
    for (int size = 2; size <= TOPK_SORT; size <<= 1) {
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            __syncthreads();
            for (int t = threadIdx.x; t < TOPK_SORT / 2; t += blockDim.x) {
                const int lo = 2 * t - (t & (stride - 1));
                const int hi = lo + stride;
                const bool desc = ((lo & size) == 0);
                const uint64_t a = k[lo], b = k[hi];
                if ((a < b) == desc) { k[lo] = b; k[hi] = a; }
            }
        }
    }
    __syncthreads();
}

// Top `topk` keys of each TOPK_SORT-sized slice. mode 0: slice of logits
// (key built from value and row), mode 1: slice of candidate keys.
__global__ __launch_bounds__(1024) void k_topk_slice(const float *__restrict__ logits,
                                                     const uint64_t *__restrict__ cand_in,
                                                     int64_t count, int mode, int topk,
                                                     uint64_t *__restrict__ cand_out) {
    __shared__ uint64_t keys[TOPK_SORT];
    const int64_t base = (int64_t)blockIdx.x * TOPK_SORT;
    for (int i = threadIdx.x; i < TOPK_SORT; i += blockDim.x) {
        const int64_t g = base + i;
        uint64_t v = 0;
        if (g < count) v = mode == 0 ? argkey(logits[g], g) : cand_in[g];
        keys[i] = v;
    }
    bitonic_desc(keys);
    for (int i = threadIdx.x; i < topk; i += blockDim.x)
        cand_out[(int64_t)blockIdx.x * topk + i] = keys[i];
}

// argmax from the GEMV's per-workgroup maxima; decode the final top-k.
__global__ __launch_bounds__(256) void k_lmhead_finalize(const uint64_t *__restrict__ partial,
                                                         int nparts, const float *__restrict__ logits,
                                                         const uint64_t *__restrict__ topkeys, int topk,
                                                         int32_t *__restrict__ argmax,
                                                         int32_t *__restrict__ topk_idx,
                                                         float *__restrict__ topk_val) {
    __shared__ uint64_t red[256];
    uint64_t m = 0;
    for (int i = threadIdx.x; i < nparts; i += blockDim.x) m = partial[i] > m ? partial[i] : m;
    red[threadIdx.x] = m;
    __syncthreads();
    for (int s = 128; s > 0; s >>= 1) {
        if (threadIdx.x < s && red[threadIdx.x + s] > red[threadIdx.x]) red[threadIdx.x] = red[threadIdx.x + s];
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        int32_t best = (int32_t)(0xffffffffu - (uint32_t)(red[0] & 0xffffffffu));
        const float l0 = logits[0];
        if (l0 != l0) best = 0;                        // sample_argmax: v = NaN never loses
        *argmax = best;
    }
    for (int i = threadIdx.x; i < topk; i += blockDim.x) {
        const int32_t idx = (int32_t)(0xffffffffu - (uint32_t)(topkeys[i] & 0xffffffffu));
        topk_idx[i] = idx;
        topk_val[i] = logits[idx];
    }
}

static int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

size_t lmhead_cand_bytes(int64_t n, int topk) {
    // argmax partials (<= 4096 workgroups) + two ping-pong candidate arrays
    const int64_t c1 = cdiv(n, TOPK_SORT) * (topk > 0 ? topk : 1);
    return (size_t)(4096 + 2 * c1 + 64) * sizeof(uint64_t);
}

hipError_t launch_lmhead(const uint8_t *w, int64_t n, int64_t k, const uint8_t *xq, int topk,
                         float *logits, int32_t *argmax, int32_t *topk_idx, float *topk_val,
                         void *cand, int fused, hipStream_t s) {
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
    uint64_t *partial = reinterpret_cast<uint64_t *>(cand);
    uint64_t *c1 = partial + 4096;
    uint64_t *c2 = c1 + cdiv(n, TOPK_SORT) * (topk > 0 ? topk : 1) + 32;
    int grid = 0;
    hipError_t e = launch_gemv_impl(a, 4096, partial, &grid, s);
    if (e != hipSuccess) return e;
    const uint64_t *top = c1;
    if (topk > 0) {
        int64_t count = n;
        int mode = 0;
        const uint64_t *in = nullptr;
        uint64_t *out = c1;
        do {
            const int64_t slices = cdiv(count, TOPK_SORT);
            hipLaunchKernelGGL(k_topk_slice, dim3((unsigned)slices), dim3(1024), 0, s, logits, in,
                               count, mode, topk, out);
            if ((e = hipGetLastError()) != hipSuccess) return e;
            top = out;
            count = slices * topk;
            in = out;
            out = (out == c1) ? c2 : c1;
            mode = 1;
            if (slices == 1) break;
        } while (true);
    }
    hipLaunchKernelGGL(k_lmhead_finalize, dim3(1), dim3(256), 0, s, partial, grid, logits, top,
                       topk, argmax, topk_idx, topk_val);
    return hipGetLastError();
}

}  // namespace qk
