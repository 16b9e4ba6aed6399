// qk_gemv.hip -- decode GEMV over native GGUF blocks (gfx950).
//
// One kernel serves every decode matmul: a launch carries up to 16
// descriptors (type, W, xq, y), so a layer's projections go out as one
// dispatch. A 256-thread workgroup computes row tiles of one descriptor
// (grid-stride over tiles).
//
// Loads. All weight loads are buffer loads whose range check covers the
// wave's current work item (rows of one tile), so no lane needs a guard.
// The wave reads its item with lane-contiguous 16-byte loads (each load
// instruction covers 1 KB of consecutive bytes, non-temporal) and passes
// it through a wave-private LDS window, from which lanes read their block
// fields at any alignment (Q6_K's 210-byte and Q8_0's 34-byte blocks
// included). For Q4_K / Q5_K this replaced per-lane loads of each block's
// fields straight into registers: 5.89 against 5.35 TB/s on a 144 MB
// Q4_K stream, 4.45 against 4.70 us for the config-1 set.
// Loads run one work item ahead of the arithmetic.
//
// Arithmetic. An aligned group of 4 lanes owns one 256-element super-block:
// each lane takes 32 quant bytes and runs v_dot4 against the activation
// bytes they meet, which it loads straight from the Q8_K row into
// registers (every workgroup reads the same row, so these loads hit the
// L2 after the first); the group sums its int32 partials with DPP. The
// super-block terms of a row are added in block order by one lane, so the
// float sum rounds exactly as the reference's sequential `sum += term`
// (simd/quants.h:305, simd/avx.c:467).
//
// Q8_0 activation rows are staged once per workgroup into LDS
// (qs[nb][32] | d[nb]).
#include "qk_dev.h"
#include "qk_kernels.h"

namespace qk {

// Range-checked view of an activation row: loads past `bytes` read zeros.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t act_rsrc(const uint8_t *xq, int bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(xq), 0, bytes, 0x00020000);
}

// Workgroup barrier that orders LDS only: it waits for the LDS stores
// before it, not for global loads still in flight.
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Q8_0 activation row: qs[nb][32] | d[nb] (fp16 widened once).
__device__ __forceinline__ void stage_q80(const uint8_t *__restrict__ xq, int nb, uint8_t *lds) {
    uint16_t *qs = reinterpret_cast<uint16_t *>(lds);
    float *d = reinterpret_cast<float *>(lds + nb * 32);
    const int tot = nb * 17;
    for (int i0 = threadIdx.x; i0 < tot; i0 += 4 * blockDim.x) {
        uint32_t v[4];
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const int i = i0 + u * (int)blockDim.x;
            if (i < tot) v[u] = ld_u16(xq + 2 * i);
        }
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const int i = i0 + u * (int)blockDim.x;
            if (i < tot) {
                const int b = i / 17, r = i - b * 17;
                if (r == 0) d[b] = h2f(v[u]);
                else qs[b * 16 + r - 1] = (uint16_t)v[u];
            }
        }
    }
}

// fp32 activation rows (hip_matvec_group_f32): the workgroup quantizes the
// row it needs into LDS itself, bit for bit as the quantize launches would.
// Q8_K blocks sit at a QXB-byte stride with the quants 16-byte aligned:
// d @0 | qs[256] @16 | bsums[16] @272. Every wave of the workgroup calls
// these (whole waves: the block quantizers use ballots and DPP).
#define QXB 304
__device__ __forceinline__ void stage_q8k_f32(const float *__restrict__ x, int nb, uint8_t *lds) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    for (int b = wave; b < nb; b += 4) {
        const float4 v = *(const QK_GLOBAL float4 *)(x + b * QK_K + 4 * lane);
        const float e[4] = {v.x, v.y, v.z, v.w};
        uint32_t packed, bs;
        float d;
        q8k_block_wave(e, lane, packed, d, bs);
        uint8_t *o = lds + b * QXB;
        *(QK_LDS uint32_t *)(o + 16 + 4 * lane) = packed;
        if ((lane & 7) == 0) *(QK_LDS uint32_t *)(o + 272 + 4 * (lane >> 3)) = bs;
        if (lane == 0) *(QK_LDS float *)(o) = d;
    }
}
// Q8_0: the layout stage_q80 writes, qs[nb][32] | d[nb] (d rounded to
// fp16 as the stored block holds it, then widened); each half-wave
// quantizes one block.
__device__ __forceinline__ void stage_q80_f32(const float *__restrict__ x, int nb, uint8_t *lds) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    float *d_out = reinterpret_cast<float *>(lds + nb * 32);
    for (int b0 = 2 * wave; b0 < nb; b0 += 8) {
        const int b = b0 + (lane >> 5), l = lane & 31;
        const float v = b < nb ? *(const QK_GLOBAL float *)(x + b * QK8_0 + l) : 0.0f;
        int32_t q;
        float d;
        q80_block_half(v, q, d);
        if (b < nb) {
            *(QK_LDS uint8_t *)(lds + b * 32 + l) = (uint8_t)(q & 0xff);
            if (l == 0) *(QK_LDS float *)(d_out + b) = h2f(f2h(d));
        }
    }
}

#define M4 0x0F0F0F0Fu

__device__ __forceinline__ int32_t dot16(uint32_t w0, uint32_t w1, uint32_t w2, uint32_t w3,
                                         const uint4 a, int32_t c) {
    int32_t s = dot4(w0, a.x, c);
    s = dot4(w1, a.y, s);
    s = dot4(w2, a.z, s);
    return dot4(w3, a.w, s);
}

// ---- LDS reads ---------------------------------------------------------------
__device__ __forceinline__ uint4 lds16(const uint8_t *p) {          // 16-B aligned
    return *(const QK_LDS uint4 *)(p);
}
__device__ __forceinline__ uint32_t lds32(const uint8_t *p) {       // 4-B aligned
    return *(const QK_LDS uint32_t *)(p);
}
__device__ __forceinline__ uint32_t lds_u16(const uint8_t *p) {     // 2-B aligned
    return *(const QK_LDS uint16_t *)(p);
}

__device__ __forceinline__ int32_t sum4(int32_t v) {
    v += dpp_xor1(v);
    v += dpp_xor2(v);
    return v;
}

// ---- wave-contiguous weight staging -------------------------------------------
// A wave item is the byte range [w + s, w + e). The wave loads its 16-byte
// aligned superset (aligned in absolute address): piece p (16 bytes) goes
// to lane p % 64 of load u = p / 64. The superset never reaches a 4 KB page
// that the range itself does not touch, since pages are 16-byte aligned.
// An item is at most 16 super-blocks (16 x 210 B), 4 Q8_0 rows of 32
// blocks (4 x 1088 B) or 64 Q8_0 blocks (64 x 34 B), plus 30 bytes of
// alignment slack. A wave loads NL x 1 KB (NL = 4 for the K-quants, 5 for
// Q8_0 rows) and chunk_store writes every load it issued whole, so the
// window holds 5 x 1 KB.
#define WBUF_BYTES 5120

template <int NL>
struct ChunkN {
    uint4 v[NL];
};
typedef ChunkN<4> Chunk;

struct Span {
    const uint8_t *base;   // 16-byte aligned start of the superset
    int32_t ofs;           // first byte of the item, relative to base
    int32_t npc;           // 16-byte pieces to load (0: empty item)
};

__device__ __forceinline__ Span make_span(const uint8_t *w, int64_t s, int64_t e) {
    const uintptr_t ps = reinterpret_cast<uintptr_t>(w + s);
    const uintptr_t pa = ps & ~(uintptr_t)15;
    Span sp;
    sp.base = reinterpret_cast<const uint8_t *>(pa);
    sp.ofs = (int32_t)(ps - pa);
    sp.npc = (int32_t)((reinterpret_cast<uintptr_t>(w + e) - pa + 15) >> 4);
    return sp;
}

// Buffer loads: the range check of the buffer resource (num_records =
// npc x 16) turns pieces past the item into zeros without a memory access,
// so the loads need no per-lane guard. A load whose 64 pieces all lie past
// the item is skipped (a uniform branch). The weights are read once per
// launch, so the loads carry the non-temporal cache policy (bit 1 of the
// buffer instruction's cache-policy operand on gfx950): 6.36 against
// 5.55 TB/s on the 209 MB LM head.
constexpr int W_NT = 2;
template <int NL>
__device__ __forceinline__ void chunk_load(ChunkN<NL> &c, const Span &sp, int lane) {
    const __amdgpu_buffer_rsrc_t r =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(sp.base), 0, sp.npc * 16, 0x00020000);
#pragma unroll
    for (int u = 0; u < NL; u++) {
        if (u * 64 < sp.npc) {
            const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, lane * 16, u * 1024, W_NT);
            c.v[u] = make_uint4(v[0], v[1], v[2], v[3]);
        }
    }
}

// Every load issued, whatever the item's length (pieces past it read
// zeros), so the wait counts of a loop that keeps two items in flight are
// known at compile time.
template <int NL>
__device__ __forceinline__ void chunk_load_all(ChunkN<NL> &c, const Span &sp, int lane) {
    const __amdgpu_buffer_rsrc_t r =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(sp.base), 0, sp.npc * 16, 0x00020000);
#pragma unroll
    for (int u = 0; u < NL; u++) {
        const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, lane * 16, u * 1024, W_NT);
        c.v[u] = make_uint4(v[0], v[1], v[2], v[3]);
    }
}

// Pieces past the item hold zeros from the range-checked loads; storing
// them stays inside the window.
template <int NL>
__device__ __forceinline__ void chunk_store(const ChunkN<NL> &c, uint8_t *wb, const Span &sp, int lane) {
#pragma unroll
    for (int u = 0; u < NL; u++)
        if (u * 64 < sp.npc) *(QK_LDS uint4 *)(wb + 1024 * u + 16 * lane) = c.v[u];
}

// Orders a wave's LDS accesses around a hand-off between its lanes. LDS
// executes one wave's instructions in order, so no wait is needed; the
// fences keep the compiler from moving accesses across.
__device__ __forceinline__ void wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Scales and mins of sub-blocks 2j and 2j+1 (q4k_get_scale_min,
// simd/quants.h:215-224) without branches: lanes j < 2 and j >= 2 take
// different forms, and a branch would run both under lane masks.
__device__ __forceinline__ void scale_min_pair(uint32_t s0, uint32_t s1, uint32_t s2, int j, int32_t &sc0,
                                               int32_t &m0, int32_t &sc1, int32_t &m1) {
    const bool hi = j >= 2;
    const uint32_t sh0 = 16u * (uint32_t)(j & 1), sh1 = sh0 + 8u;   // byte (2j) & 3, (2j+1) & 3
    auto one = [&](uint32_t sh, int32_t &sc, int32_t &m) {
        const uint32_t lo_sc = __builtin_amdgcn_ubfe(s0, sh, 6), lo_m = __builtin_amdgcn_ubfe(s1, sh, 6);
        const uint32_t hi_sc = __builtin_amdgcn_ubfe(s2, sh, 4) | (__builtin_amdgcn_ubfe(s0, sh + 6, 2) << 4);
        const uint32_t hi_m = __builtin_amdgcn_ubfe(s2, sh + 4, 4) | (__builtin_amdgcn_ubfe(s1, sh + 6, 2) << 4);
        sc = (int32_t)(hi ? hi_sc : lo_sc);
        m = (int32_t)(hi ? hi_m : lo_m);
    };
    one(sh0, sc0, m0);
    one(sh1, sc1, m1);
}

// ---- per-super-block fields and terms -------------------------------------------
// Lane j (0..3) of a group holds its 32 quant bytes of the super-block and
// the header, read from the wave's LDS window.
template <int T> struct Raw;
template <> struct Raw<12> { uint4 hdr, q0, q1; };
template <> struct Raw<13> { uint4 hdr, q0, q1, h0, h1; };
template <> struct Raw<14> { uint32_t l[9], h[9], sh, sc, sc2, d; };

// Q6_K (simd/quants.h:356-402). Lane j = 2h + qq holds ql bytes
// [32j, 32j+32) (positions l = 0..31 of half h, quarter qq): the low
// nibble is element 128h + 32qq + l, the high nibble element +64; the two
// top bits come from qh[32h + l] bits 2qq and 2qq+4. Sub-blocks
// 8h+2qq+{0,1} (low) and +4 (high). Each lane folds its share of
// isum - 32*isum_mins, exact in int32, so one reduction suffices. 210-byte
// blocks sit at even offsets: 32-byte runs are read as aligned 36-byte
// windows (inside the block: the last ends at byte 196) and funnel-shifted.
__device__ __forceinline__ void read_sb(Raw<14> &r, const uint8_t *wb, int off, int j) {
    const int h = j >> 1, qq = j & 1;
    const uint32_t sh = (uint32_t)off & 3u;
    r.sh = sh;
    const uint8_t *wl = wb + off + 32 * j - sh;
    const uint8_t *wh = wb + off + 128 + 32 * h - sh;
#pragma unroll
    for (int i = 0; i < 9; i++) {
        r.l[i] = lds32(wl + 4 * i);
        r.h[i] = lds32(wh + 4 * i);
    }
    const int s = 8 * h + 2 * qq;
    r.sc = lds_u16(wb + off + 192 + s);
    r.sc2 = lds_u16(wb + off + 196 + s);
    r.d = lds_u16(wb + off + 208);
}

// Q4_K / Q5_K blocks (144 / 176 bytes, so 16-byte aligned in the window):
// the header, then lane j's 32 quant bytes (and Q5_K's 32 qh bytes).
__device__ __forceinline__ void read_sb(Raw<12> &r, const uint8_t *wb, int off, int j) {
    r.hdr = *(const QK_LDS uint4 *)(wb + off);
    r.q0 = *(const QK_LDS uint4 *)(wb + off + 16 + 32 * j);
    r.q1 = *(const QK_LDS uint4 *)(wb + off + 32 + 32 * j);
}
__device__ __forceinline__ void read_sb(Raw<13> &r, const uint8_t *wb, int off, int j) {
    r.hdr = *(const QK_LDS uint4 *)(wb + off);
    r.h0 = *(const QK_LDS uint4 *)(wb + off + 16);
    r.h1 = *(const QK_LDS uint4 *)(wb + off + 32);
    r.q0 = *(const QK_LDS uint4 *)(wb + off + 48 + 32 * j);
    r.q1 = *(const QK_LDS uint4 *)(wb + off + 64 + 32 * j);
}

// ---- activation operands straight from the Q8_K row -----------------------
// Block b of the row is 292 bytes: d (f32) | qs[256] | bsums[16] (i16).
// Each lane loads the activation bytes its weights meet with range-checked
// buffer loads (a lane of a super-block past the row end reads zeros and
// its term is never added). Every workgroup reads the same row, so these
// loads hit the L2 after the first.
// Q4_K / Q5_K lane j: qs[64j, 64j+64), bsums 4j..4j+3 (pairs 2j, 2j+1), d.
struct ActK { uint4 a0, a1, a2, a3; uint32_t bs0, bs1; float d; };
__device__ __forceinline__ void load_act(ActK &x, __amdgpu_buffer_rsrc_t r, int b, int j) {
    const int o = b * Q8K_BYTES;
    x.a0 = bl128(r, o + 4 + 64 * j);
    x.a1 = bl128(r, o + 20 + 64 * j);
    x.a2 = bl128(r, o + 36 + 64 * j);
    x.a3 = bl128(r, o + 52 + 64 * j);
    x.bs0 = bl32(r, o + 260 + 8 * j);
    x.bs1 = bl32(r, o + 264 + 8 * j);
    x.d = __uint_as_float(bl32(r, o));
}
// Q6_K lane j = 2h + qq, s = 8h + 2qq: qs of sub-blocks s, s+1 and s+4,
// s+5, bsums s, s+1 and s+4, s+5, d.
struct Act6 { uint4 a0, a1, a4, a5; uint32_t bl, bh; float d; };
__device__ __forceinline__ void load_act(Act6 &x, __amdgpu_buffer_rsrc_t r, int b, int j) {
    const int o = b * Q8K_BYTES, s = 8 * (j >> 1) + 2 * (j & 1);
    x.a0 = bl128(r, o + 4 + 16 * s);
    x.a1 = bl128(r, o + 20 + 16 * s);
    x.a4 = bl128(r, o + 68 + 16 * s);
    x.a5 = bl128(r, o + 84 + 16 * s);
    x.bl = bl32(r, o + 260 + 2 * s);
    x.bh = bl32(r, o + 268 + 2 * s);
    x.d = __uint_as_float(bl32(r, o));
}
// The same fields from a row the workgroup quantized into LDS (QXB layout).
__device__ __forceinline__ void load_act_lds(ActK &x, const uint8_t *l, int b, int j) {
    const uint8_t *o = l + b * QXB;
    x.a0 = *(const QK_LDS uint4 *)(o + 16 + 64 * j);
    x.a1 = *(const QK_LDS uint4 *)(o + 32 + 64 * j);
    x.a2 = *(const QK_LDS uint4 *)(o + 48 + 64 * j);
    x.a3 = *(const QK_LDS uint4 *)(o + 64 + 64 * j);
    x.bs0 = *(const QK_LDS uint32_t *)(o + 272 + 8 * j);
    x.bs1 = *(const QK_LDS uint32_t *)(o + 276 + 8 * j);
    x.d = *(const QK_LDS float *)(o);
}
__device__ __forceinline__ void load_act_lds(Act6 &x, const uint8_t *l, int b, int j) {
    const uint8_t *o = l + b * QXB;
    const int s = 8 * (j >> 1) + 2 * (j & 1);
    x.a0 = *(const QK_LDS uint4 *)(o + 16 + 16 * s);
    x.a1 = *(const QK_LDS uint4 *)(o + 32 + 16 * s);
    x.a4 = *(const QK_LDS uint4 *)(o + 80 + 16 * s);
    x.a5 = *(const QK_LDS uint4 *)(o + 96 + 16 * s);
    x.bl = *(const QK_LDS uint32_t *)(o + 272 + 2 * s);
    x.bh = *(const QK_LDS uint32_t *)(o + 280 + 2 * s);
    x.d = *(const QK_LDS float *)(o);
}
template <int T> struct ActOf { typedef ActK type; };
template <> struct ActOf<14> { typedef Act6 type; };

__device__ __forceinline__ int32_t dot32r(const uint32_t (&w)[8], const uint4 a0, const uint4 a1) {
    int32_t s = dot4(w[0], a0.x, 0);
    s = dot4(w[1], a0.y, s);
    s = dot4(w[2], a0.z, s);
    s = dot4(w[3], a0.w, s);
    s = dot4(w[4], a1.x, s);
    s = dot4(w[5], a1.y, s);
    s = dot4(w[6], a1.z, s);
    return dot4(w[7], a1.w, s);
}
__device__ __forceinline__ int32_t pair_of(uint32_t v) {
    return (int32_t)(int16_t)(v & 0xffffu) + (int32_t)(int16_t)(v >> 16);
}

// Q4_K (simd/quants.h:267-306): lane j holds chunk c = j, qs[32j..32j+32):
// low nibbles pair with q8[64j..64j+32) under scale 2j, high nibbles with
// q8[64j+32..64j+64) under scale 2j+1; mins 2j, 2j+1 meet bsum pairs 2j,
// 2j+1.
template <bool FUSED>
__device__ __forceinline__ float term_sb(const Raw<12> &r, const ActK &x, int j) {
    const uint32_t q[8] = {r.q0.x, r.q0.y, r.q0.z, r.q0.w, r.q1.x, r.q1.y, r.q1.z, r.q1.w};
    uint32_t lo[8], hi[8];
#pragma unroll
    for (int i = 0; i < 8; i++) {
        lo[i] = q[i] & M4;
        hi[i] = (q[i] >> 4) & M4;
    }
    const int32_t slo = dot32r(lo, x.a0, x.a1), shi = dot32r(hi, x.a2, x.a3);
    int32_t sc0, m0, sc1, m1;
    scale_min_pair(r.hdr.y, r.hdr.z, r.hdr.w, j, sc0, m0, sc1, m1);
    const int32_t isum = sum4(__mul24(slo, sc0) + __mul24(shi, sc1));
    const int32_t mins = sum4(__mul24(m0, pair_of(x.bs0)) + __mul24(m1, pair_of(x.bs1)));
    return kterm<FUSED>(x.d, r.hdr.x & 0xffffu, r.hdr.x >> 16, isum, mins);
}
// Q5_K (simd/quants.h:310-351): as Q4_K plus bit 2j / 2j+1 of qh[l].
template <bool FUSED>
__device__ __forceinline__ float term_sb(const Raw<13> &r, const ActK &x, int j) {
    const uint32_t q[8] = {r.q0.x, r.q0.y, r.q0.z, r.q0.w, r.q1.x, r.q1.y, r.q1.z, r.q1.w};
    const uint32_t qh[8] = {r.h0.x, r.h0.y, r.h0.z, r.h0.w, r.h1.x, r.h1.y, r.h1.z, r.h1.w};
    // rotations that bring bit 2j (2j+1) of every byte to its bit 4, where
    // the fifth bit belongs; the bit moves by at most 3, inside its byte
    const uint32_t r0 = (uint32_t)(2 * j - 4) & 31u, r1 = (uint32_t)(2 * j - 3) & 31u;
    uint32_t lo[8], hi[8];
#pragma unroll
    for (int i = 0; i < 8; i++) {
        lo[i] = (q[i] & M4) | (__builtin_amdgcn_alignbit(qh[i], qh[i], r0) & 0x10101010u);
        hi[i] = ((q[i] >> 4) & M4) | (__builtin_amdgcn_alignbit(qh[i], qh[i], r1) & 0x10101010u);
    }
    const int32_t slo = dot32r(lo, x.a0, x.a1), shi = dot32r(hi, x.a2, x.a3);
    int32_t sc0, m0, sc1, m1;
    scale_min_pair(r.hdr.y, r.hdr.z, r.hdr.w, j, sc0, m0, sc1, m1);
    const int32_t isum = sum4(__mul24(slo, sc0) + __mul24(shi, sc1));
    const int32_t mins = sum4(__mul24(m0, pair_of(x.bs0)) + __mul24(m1, pair_of(x.bs1)));
    return kterm<FUSED>(x.d, r.hdr.x & 0xffffu, r.hdr.x >> 16, isum, mins);
}
// Q6_K: the lane's share of isum - 32*isum_mins over sub-blocks s, s+1,
// s+4, s+5 (see read_sb), exact in int32. Each sub-block's dot chain
// starts from -32*bsum, so it yields sum((q - 32) * a) directly; the seed
// depends on the activations only and is formed once per wave when they
// stay put. |chain| < 2^18 fits the 24-bit multiply.
template <bool FUSED>
__device__ __forceinline__ float term_sb(const Raw<14> &r, const Act6 &x, int j) {
    const int qq = j & 1;
    const uint32_t sh = r.sh, sb = 8 * sh + 2 * qq;
    uint32_t lo[8], hi[8];
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const uint32_t ql = __builtin_amdgcn_alignbyte(r.l[i + 1], r.l[i], sh);
        // one funnel shift aligns the qh bytes and brings the lane's bit
        // pairs to bits 0-1 (low nibble's) and 4-5 (high nibble's) of
        // each byte; the mask drops the bits shifted in from the next byte
        const uint32_t qh = __builtin_amdgcn_alignbit(r.h[i + 1], r.h[i], sb) & 0x33333333u;
        lo[i] = (ql & M4) | ((qh << 4) & ~M4);
        hi[i] = ((ql >> 4) & M4) | (qh & ~M4);
    }
    const int32_t b0 = (int16_t)(x.bl & 0xffffu), b1 = (int16_t)(x.bl >> 16);
    const int32_t b4 = (int16_t)(x.bh & 0xffffu), b5 = (int16_t)(x.bh >> 16);
    const int32_t d0 = dot16(lo[0], lo[1], lo[2], lo[3], x.a0, -32 * b0);
    const int32_t d1 = dot16(lo[4], lo[5], lo[6], lo[7], x.a1, -32 * b1);
    const int32_t d4 = dot16(hi[0], hi[1], hi[2], hi[3], x.a4, -32 * b4);
    const int32_t d5 = dot16(hi[4], hi[5], hi[6], hi[7], x.a5, -32 * b5);
    const int32_t sc0 = (int32_t)(int8_t)(r.sc & 0xffu), sc1 = (int32_t)(int8_t)(r.sc >> 8);
    const int32_t sc4 = (int32_t)(int8_t)(r.sc2 & 0xffu), sc5 = (int32_t)(int8_t)(r.sc2 >> 8);
    const int32_t v = __mul24(d0, sc0) + __mul24(d1, sc1) + __mul24(d4, sc4) + __mul24(d5, sc5);
    const int32_t tot = sum4(v);
    return q6term(x.d, r.d, tot);
}

// Device-side descriptor: 64 bytes, fetched by one scalar load once a
// workgroup knows its descriptor index.
struct KDesc {
    const uint8_t *w;
    const uint8_t *xq;
    float *y;
    int32_t n;
    int32_t type;
    int32_t nb;
    int32_t p;
    int32_t rows_per_tile;
    int32_t ntiles;
    int32_t nwg;
    int32_t lds_act;
    int32_t wg0;
    int32_t xf32;          // 1: xq holds the fp32 row; the workgroup quantizes it into LDS
};
static_assert(sizeof(KDesc) == 64, "KDesc is one 64-byte scalar load");

struct alignas(64) KArgs {
    KDesc d[QK_GROUP_MAX_DEV];
};

// Monotone 64-bit key: larger logit first, lower index on ties; -0 == +0
// and NaN below everything (sample_argmax never picks a NaN).
__device__ __forceinline__ uint64_t argkey(float v, int64_t row) {
    uint32_t b = __float_as_uint(v);
    if (v == 0.0f) b = 0;
    uint32_t key = (v != v) ? 0u : ((b & 0x80000000u) ? ~b : (b | 0x80000000u));
    return ((uint64_t)key << 32) | (uint64_t)(0xffffffffu - (uint32_t)row);
}

// The P super-block terms of a row, from the first lane of each of its P
// four-lane groups, into the row's first lane (the only lane that adds
// and stores them, in order). P = 4: the groups sit 4 lanes apart in one
// 16-lane row, so DPP row_shl moves them. P = 16 (one row per wave):
// row_shl inside each 16-lane row, then the four rows' first lanes read
// as uniform values. P = 8 (two rows per wave) uses ds_bpermute.
template <int P>
__device__ __forceinline__ void gather_terms(float (&tg)[P], float t, int src0) {
    if constexpr (P == 4) {
        tg[0] = t;
        tg[1] = __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(t), 0x104, 0xF, 0xF, true));
        tg[2] = __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(t), 0x108, 0xF, 0xF, true));
        tg[3] = __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(t), 0x10C, 0xF, 0xF, true));
    } else if constexpr (P == 16) {
        // one row per wave: each 16-lane DPP row gathers its four groups
        // into its first lane, which the wave then reads as uniform values
        const int v0 = __float_as_int(t);
        const int v1 = __builtin_amdgcn_mov_dpp(v0, 0x104, 0xF, 0xF, true);
        const int v2 = __builtin_amdgcn_mov_dpp(v0, 0x108, 0xF, 0xF, true);
        const int v3 = __builtin_amdgcn_mov_dpp(v0, 0x10C, 0xF, 0xF, true);
#pragma unroll
        for (int r = 0; r < 4; r++) {
            tg[4 * r + 0] = __int_as_float(__builtin_amdgcn_readlane(v0, 16 * r));
            tg[4 * r + 1] = __int_as_float(__builtin_amdgcn_readlane(v1, 16 * r));
            tg[4 * r + 2] = __int_as_float(__builtin_amdgcn_readlane(v2, 16 * r));
            tg[4 * r + 3] = __int_as_float(__builtin_amdgcn_readlane(v3, 16 * r));
        }
    } else {
#pragma unroll
        for (int g2 = 0; g2 < P; g2++) tg[g2] = __shfl(t, src0 + 4 * g2);
    }
}

// K-quant rows handled by this workgroup (the LDS-window path): tiles
// lw, lw+nwg, ... of 4 waves x 16/P rows. A row's P = 2^LP groups each take
// one super-block of a step (P super-blocks); the P terms of a step are
// gathered into the row's first lane and added to the row sum in
// super-block order. A wave item (tile, step) is one contiguous range of
// W: the wave's 16/P whole rows when a row fits one step (nb <= P), else P
// super-blocks of its one row (P = 16). Items are pipelined one deep: item
// i+1's loads are issued before item i is reduced; the activation
// operands' loads go out before the first item's. Item offsets are
// 32-bit: the API limits a matrix to 4 GB.
//
// LM (the LM-head kernel, whose register budget allows 4 waves per SIMD;
// it runs 2): waves of many one-item rows alternate two register sets, so
// the loads of the next item are in flight while the wave waits for the
// current one's. The general loop must instead wait for all loads before
// it moves the look-ahead registers into place.
template <int TYPE, int LP, bool FUSED, bool LM, bool XF>
__device__ __forceinline__ void run_kq(const KDesc &D, int lw, int nwg, uint8_t *lds, uint64_t &best, bool keys) {
    constexpr int BB = TYPE == 12 ? Q4K_BYTES : (TYPE == 13 ? Q5K_BYTES : Q6K_BYTES);
    constexpr int P = 1 << LP;
    constexpr int RPW = 16 >> LP;                      // rows per wave item
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int grp = lane >> 2, j = lane & 3;
    const int team = grp >> LP, g = grp & (P - 1);
    const int nb = D.nb, ntiles = D.ntiles, n = D.n;
    const int niter = (nb + P - 1) >> LP;
    const uint32_t rowb = (uint32_t)nb * BB;
    const uint8_t *__restrict__ w = D.w;
    float *__restrict__ y = D.y;
    uint8_t *wb = lds + D.lds_act + wave * WBUF_BYTES;
    const int src0 = team * P * 4;
    const int lofs = (team * nb + g) * BB;             // block offset inside the item
    auto span = [&](int t, int i) -> Span {
        const int r0 = t * (4 * RPW) + wave * RPW;
        uint32_t len;
        if (niter == 1) {
            const int nr = (n - r0 < RPW) ? n - r0 : RPW;
            len = (uint32_t)nr * rowb;
        } else {
            const int nbl = (nb - i * P < P) ? nb - i * P : P;
            len = (uint32_t)nbl * BB;
        }
        if (t >= ntiles || r0 >= n) len = 0;
        const uint32_t s0 = (uint32_t)r0 * rowb + (uint32_t)(i * P * BB);
        const uint32_t a0 = s0 & ~15u;
        Span sp;
        sp.base = w + a0;
        sp.ofs = (int32_t)(s0 - a0);
        sp.npc = len ? (int32_t)((s0 + len - a0 + 15) >> 4) : 0;
        return sp;
    };
    // activation operands of super-block g first (those of every item
    // when a row is one item), then the first item's weights
    const __amdgpu_buffer_rsrc_t ar = act_rsrc(D.xq, nb * Q8K_BYTES);
    // fp32 row: quantized into LDS after the first item's loads are issued
    const uint8_t *xl = XF ? lds : nullptr;
    typename ActOf<TYPE>::type xa;
    if (!xl) load_act(xa, ar, g, j);
    int xit = 0;
    int tile = lw, it = 0;
    Span sp = span(tile, it);
    Chunk cur;
    chunk_load(cur, sp, lane);
    if (xl) {
        stage_q8k_f32(reinterpret_cast<const float *>(D.xq), nb, lds);
        lds_barrier();
        load_act_lds(xa, xl, g, j);
    }
    int ntile = tile, nit = it + 1;
    if (nit == niter) { nit = 0; ntile += nwg; }
    Span nsp = span(ntile, nit);                       // computed while the loads are in flight
    float sum = 0.0f;
    // Argmax keys: each storing lane keeps its first-index maximum as a
    // value and a row, and forms the 64-bit key once at the end. Its rows
    // ascend, so only a strictly larger value replaces the one held; bv
    // starts as NaN (no row yet) and a NaN row is never taken.
    float bv = __int_as_float(0x7fc00000);
    int brow = -1;
    auto finish = [&]() __attribute__((always_inline)) {
        if (keys && brow >= 0) {
            const uint64_t k = argkey(bv, brow);
            best = k > best ? k : best;
        }
    };
    // item (tile, it) from registers c (range sp): through the window, the
    // term, gathered into the row's first lane, which stores the row after
    // its last item
    auto item = [&](const Chunk &c, const Span &sp, int tile, int it) __attribute__((always_inline)) {
        chunk_store(c, wb, sp, lane);
        wave_sync();
        // Lanes of a block past the row end or of a row past n compute a
        // term from in-range LDS bytes that is replaced by +0.0 or never
        // stored.
        Raw<TYPE> r;
        read_sb(r, wb, sp.ofs + lofs, j);
        if (it != xit) {                               // rows of several items: next super-blocks
            if (xl) load_act_lds(xa, xl, it * P + g, j);
            else load_act(xa, ar, it * P + g, j);
            xit = it;
        }
        // A group past the row end contributes +0.0: the sum starts at
        // +0.0 and can never become -0.0, so adding +0.0 leaves it as is.
        const int lim = (nb - it * P < P) ? nb - it * P : P;
        const float t0 = term_sb<FUSED>(r, xa, j);
        const float t = g < lim ? t0 : 0.0f;
        float tg[P];
        gather_terms<P>(tg, t, src0);
#pragma unroll
        for (int g2 = 0; g2 < P; g2++) sum += tg[g2];
        if (it == niter - 1) {
            const int row = tile * (4 * RPW) + wave * RPW + team;
            if (FUSED) sum = bcast8(sum);
            if (row < n && g == 0 && j == 0) {
                *(QK_GLOBAL float *)(y + row) = sum;
                if (keys) {
                    const bool take = !(sum <= bv) && sum == sum;
                    bv = take ? sum : bv;
                    brow = take ? row : brow;
                }
            }
            sum = 0.0f;
        }
        wave_sync();                                   // window reads done before the next store
    };
    if (ntile >= ntiles) {                             // one item (a decode launch): no look-ahead
        item(cur, sp, tile, it);
        finish();
        return;
    }
    if constexpr (LM) {
        if (niter == 1) {
            Chunk nxt;
            while (true) {
                chunk_load_all(nxt, nsp, lane);        // past the last tile: zeros, never stored
                item(cur, sp, tile, 0);
                sp = nsp;
                tile = ntile;
                ntile += nwg;
                nsp = span(ntile, 0);
                if (tile >= ntiles) break;
                chunk_load_all(cur, nsp, lane);
                item(nxt, sp, tile, 0);
                sp = nsp;
                tile = ntile;
                ntile += nwg;
                nsp = span(ntile, 0);
                if (tile >= ntiles) break;
            }
            finish();
            return;
        }
    }
    while (tile < ntiles) {
        Chunk nxt;
        chunk_load(nxt, nsp, lane);
        item(cur, sp, tile, it);
        cur = nxt;
        sp = nsp;
        tile = ntile;
        it = nit;
        ntile = tile;
        nit = it + 1;
        if (nit == niter) { nit = 0; ntile += nwg; }
        nsp = span(ntile, nit);
    }
    finish();
}

// Q8_0 (q8_0_dot_q8_0, simd/avx.c:65-158, simd/quants.h:244-256): one row
// per wave, in chunks of up to 64 blocks (one wave item, pipelined like the
// K-quants). Lane = slot s (bytes 4s..4s+3 of a block, the AVX lane) +
// 8 x phase; phases take blocks b = phase + 8i of the chunk. The per-block
// slot partials p and scales go back through the wave's LDS window to 8
// chain lanes, which run the reference's sequential accumulation over
// blocks:
//  fused (AVX2/VNNI): acc_s = fma((float)p_s, s_b, acc_s), then
//        ((a0+a4)+(a1+a5)) + ((a2+a6)+(a3+a7));
//  separate (scalar/AVX1): sum = sum + (float)(sum_s p_s) * s_b.
template <bool FUSED, bool XF>
__device__ __forceinline__ void run_q80(const KDesc &D, int lw, int nwg, uint8_t *lds, uint64_t &best, bool keys) {
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int s = lane & 7, ph = lane >> 3;
    const int nb = D.nb, ntiles = D.ntiles;
    const int nchunk = (nb + 63) >> 6;
    const int64_t n = D.n;
    const uint8_t *__restrict__ w = D.w;
    float *__restrict__ y = D.y;
    uint8_t *wb = lds + D.lds_act + wave * WBUF_BYTES;
    // after a chunk's raw bytes are read: 8 slots x 64 blocks of partials
    // (slot-major, so a chain lane reads contiguous 16-byte vectors) and 64
    // block scales, in the same window
    QK_LDS int32_t *xp = (QK_LDS int32_t *)(wb);
    QK_LDS float *xs = (QK_LDS float *)(xp + 64 * 8);
    auto span = [&](int t, int c) -> Span {
        const int64_t row = (int64_t)t * 4 + wave;
        if (t >= ntiles || row >= n) return Span{w, 0, 0};
        const int b1 = (c * 64 + 64 < nb) ? c * 64 + 64 : nb;
        return make_span(w, (row * nb + (int64_t)c * 64) * Q80_BYTES, (row * nb + b1) * Q80_BYTES);
    };
    int tile = lw, c = 0;
    Span sp = span(tile, c);
    Chunk cur;
    chunk_load(cur, sp, lane);
    if constexpr (XF) stage_q80_f32(reinterpret_cast<const float *>(D.xq), nb, lds);
    else stage_q80(D.xq, nb, lds);
    __syncthreads();
    const QK_LDS uint32_t *aq = (const QK_LDS uint32_t *)(lds);
    const QK_LDS float *ad = (const QK_LDS float *)(lds + nb * 32);
    float acc = 0.0f;
    while (tile < ntiles) {
        int ntile = tile, nc = c + 1;
        if (nc == nchunk) { nc = 0; ntile += nwg; }
        const Span nsp = span(ntile, nc);
        Chunk nxt;
        chunk_load(nxt, nsp, lane);
        const int64_t row = (int64_t)tile * 4 + wave;
        if (row < n) {                                 // wave-uniform
            chunk_store(cur, wb, sp, lane);
            wave_sync();
            const int c0 = c * 64;
            const int cn = (nb - c0 < 64) ? nb - c0 : 64;
            uint32_t wq[8], wd[8];
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const int bl = ph + 8 * i;
                if (bl < cn) {
                    const uint8_t *blk = wb + sp.ofs + bl * Q80_BYTES;
                    wq[i] = lds_u16(blk + 2 + 4 * s) | (lds_u16(blk + 4 + 4 * s) << 16);
                    wd[i] = lds_u16(blk);
                }
            }
            wave_sync();                               // raw reads done before xp/xs reuse the window
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
            wave_sync();
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
            wave_sync();                               // chain reads done before the next chunk
            if (c == nchunk - 1) {
                float r = acc;
                if (FUSED) {
                    r = __fadd_rn(r, swz_xor4(r));
                    r = __fadd_rn(r, swz_xor1(r));
                    r = __fadd_rn(r, swz_xor2(r));
                }
                if (lane == 0) {
                    *(QK_GLOBAL float *)(y + row) = r;
                    if (keys) {
                        const uint64_t k = argkey(r, row);
                        best = k > best ? k : best;
                    }
                }
                acc = 0.0f;
            }
        }
        cur = nxt;
        sp = nsp;
        tile = ntile;
        c = nc;
    }
}

// Q8_0 rows of 16 or 32 blocks (k = 512 or 1024; the model's Q8_0 width).
// 4 rows per wave: lane = 16r + 8h + s (row r, parity h, slot s = the AVX
// lane of bytes 4s..4s+3), 16 rows per workgroup. The wave's 4 rows are
// one contiguous range (at most 4 x 1088 B) staged through the LDS window.
// Lane (r, h, s) forms the slot partial p and the scale of the blocks of
// parity h; lane (r, 0, s) runs the reference's sequential chain over
// blocks, taking odd blocks from lane (r, 1, s) by DPP (row_shl:8):
//  fused (AVX2/VNNI): acc_s = fma((float)p_s, s_b, acc_s), then
//        ((a0+a4)+(a1+a5)) + ((a2+a6)+(a3+a7)) over the 8 slot lanes;
//  separate (scalar/AVX1): sum = sum + (float)(sum_s p_s) * s_b, the slot
//        sum by DPP inside each 8-lane group.
// Rows of 16n blocks are 16-byte multiples, so blocks sit at offsets
// 34b from a 16-byte aligned row start.
__device__ __forceinline__ int32_t dpp_shl8(int32_t v) {
    return __builtin_amdgcn_mov_dpp(v, 0x108, 0xF, 0xF, true);   // row_shl:8
}

template <int NB, bool FUSED, bool XF>
__device__ __forceinline__ void run_q80r(const KDesc &D, int lw, int nwg, uint8_t *lds, uint64_t &best, bool keys) {
    constexpr int ROWB = NB * Q80_BYTES;               // 544 or 1088
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int r = lane >> 4, h = (lane >> 3) & 1, s = lane & 7;
    const int n = D.n, ntiles = D.ntiles;
    const uint8_t *__restrict__ w = D.w;
    float *__restrict__ y = D.y;
    uint8_t *wb = lds + D.lds_act + wave * WBUF_BYTES;
    auto span = [&](int t) -> Span {
        const int r0 = t * 16 + wave * 4;
        const int nr = (n - r0 < 4) ? n - r0 : 4;
        Span sp;
        sp.base = w + (uint32_t)r0 * ROWB;
        sp.ofs = 0;
        sp.npc = (t < ntiles && nr > 0) ? nr * (ROWB / 16) : 0;
        return sp;
    };
    // activation loads (u16: qs pairs and d) first, then the weights
    constexpr int TOT = NB * 17, NR = (TOT + 255) / 256;
    const __amdgpu_buffer_rsrc_t ar = act_rsrc(D.xq, NB * Q80_BYTES);
    uint32_t av[NR];
    if constexpr (!XF) {
#pragma unroll
        for (int u = 0; u < NR; u++)
            av[u] = __builtin_amdgcn_raw_buffer_load_b16(ar, 2 * (256 * u + (int)threadIdx.x), 0, 0);
    }
    int tile = lw;
    Span sp = span(tile);
    ChunkN<5> cur;
    chunk_load(cur, sp, lane);
    if constexpr (XF) {
        // fp32 row: quantized into the same layout after the weight loads
        stage_q80_f32(reinterpret_cast<const float *>(D.xq), NB, lds);
    } else {
        // qs[NB][32] as u16 pairs | d[NB] widened to float
        uint8_t *junk = lds + D.lds_act;
#pragma unroll
        for (int u = 0; u < NR; u++) {
            const int i = 256 * u + (int)threadIdx.x;
            const int b = i / 17, q = i - b * 17;
            const uint32_t val = q == 0 ? __float_as_uint(h2f(av[u])) : av[u];
            uint8_t *dst = q == 0 ? lds + NB * 32 + 4 * b : lds + b * 32 + 2 * q - 2;
            dst = i < TOT ? dst : junk;
            if (q == 0) *(QK_LDS uint32_t *)(dst) = val;
            else *(QK_LDS uint16_t *)(dst) = (uint16_t)val;
        }
    }
    lds_barrier();
    const QK_LDS uint32_t *aq = (const QK_LDS uint32_t *)(lds);
    const QK_LDS float *ad = (const QK_LDS float *)(lds + NB * 32);
    // item `tile` from registers c (range sp): through the window, then
    // four rows' dots and one store per row
    auto item = [&](const ChunkN<5> &c, const Span &sp, int tile) __attribute__((always_inline)) {
        chunk_store(c, wb, sp, lane);
        wave_sync();
        const int nr = sp.npc / (ROWB / 16);
        const uint8_t *rowp = wb + r * ROWB;
        float acc = 0.0f;
#pragma unroll 4
        for (int i = 0; i < NB / 2; i++) {
            const int b = 2 * i + h;
            const int off = b * Q80_BYTES + 2 + 4 * s;     // 2 mod 4 for even b, 0 for odd
            const int a4 = off & ~3;
            const uint32_t x0 = lds32(rowp + a4), x1 = lds32(rowp + a4 + 4);
            const uint32_t w4 = __builtin_amdgcn_alignbyte(x1, x0, (uint32_t)(off & 3));
            const int32_t p = dot4(w4, aq[b * 8 + s], 0);
            const float sc = __fmul_rn(h2f(lds_u16(rowp + b * Q80_BYTES)), ad[b]);
            if (FUSED) {
                const float po = __int_as_float(dpp_shl8(__float_as_int((float)p)));
                const float so = __int_as_float(dpp_shl8(__float_as_int(sc)));
                acc = __builtin_fmaf((float)p, sc, acc);
                acc = __builtin_fmaf(po, so, acc);
            } else {
                const float t = __fmul_rn((float)sum8(p), sc);
                const float to = __int_as_float(dpp_shl8(__float_as_int(t)));
                acc = __fadd_rn(acc, t);
                acc = __fadd_rn(acc, to);
            }
        }
        if (FUSED) {
            acc = __fadd_rn(acc, swz_xor4(acc));
            acc = __fadd_rn(acc, swz_xor1(acc));
            acc = __fadd_rn(acc, swz_xor2(acc));
        }
        const int row = tile * 16 + wave * 4 + r;
        if (r < nr && h == 0 && s == 0) {
            *(QK_GLOBAL float *)(y + row) = acc;
            if (keys) {
                const uint64_t k = argkey(acc, row);
                best = k > best ? k : best;
            }
        }
        wave_sync();                                   // window reads done before the next store
    };
    if (tile + nwg >= ntiles) {                        // one item (a decode launch): no look-ahead
        item(cur, sp, tile);
        return;
    }
    while (tile < ntiles) {
        const int ntile = tile + nwg;
        const Span nsp = span(ntile);
        ChunkN<5> nxt;
        chunk_load(nxt, nsp, lane);
        item(cur, sp, tile);
        cur = nxt;
        sp = nsp;
        tile = ntile;
    }
}

// One launch, up to 16 descriptors. Workgroups [wg0, wg0 + nwg) of a
// launch belong to descriptor d. The first workgroup of every descriptor
// travels as 16-bit fields of the first eight arguments, which the build
// preloads into SGPRs (-amdgpu-kernarg-preload-count=8): a workgroup finds
// its descriptor without a memory round trip, then fetches the 64-byte
// descriptor with one scalar load. Kernel-argument loads are on every
// workgroup's critical path and each dependent one costs a trip to memory,
// so a search that reads wg0 descriptor by descriptor would cost one trip
// per descriptor passed.
__device__ __forceinline__ int wg0_of(uint32_t t, int hi) { return (int)(hi ? t >> 16 : t & 0xffffu); }

// LM: the LM-head instantiation (one Q6_K matrix, many items per wave),
// allowed 128 VGPRs for its two register sets; decode launches keep the
// 5-wave bound.
// XF: every descriptor's activations are fp32 rows, quantized by each
// workgroup (hip_matvec_group_f32).
template <bool FUSED, bool LM, bool XF>
__global__ __launch_bounds__(256, LM ? 4 : 5) void k_gemv(uint32_t t0, uint32_t t1, uint32_t t2, uint32_t t3,
                                              uint32_t t4, uint32_t t5, uint32_t t6, uint32_t t7,
                                              KArgs args, uint64_t *__restrict__ amax_partial,
                                              uint32_t *__restrict__ zero_ctr) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    const uint32_t tab[8] = {t0, t1, t2, t3, t4, t5, t6, t7};
    const int bx = (int)blockIdx.x;
    // di = the last descriptor whose first workgroup is <= bx (first
    // workgroups increase with the index; unused entries hold 0xffff)
    int di = 0;
#pragma unroll
    for (int i = 1; i < QK_GROUP_MAX_DEV; i++) {
        if (wg0_of(tab[i >> 1], i & 1) > bx) break;
        di = i;
    }
    // the whole descriptor in one s_load_dwordx16
    typedef uint32_t u32x16 __attribute__((ext_vector_type(16)));
    const u32x16 raw = *reinterpret_cast<const u32x16 *>(&args.d[di]);
    KDesc D;
    __builtin_memcpy(&D, &raw, sizeof(KDesc));
    const int lw = (int)blockIdx.x - D.wg0;
    uint64_t best = 0;
    const bool keys = amax_partial != nullptr;        // argmax keys (LM head) wanted
    switch (D.type) {
        case 12:
            if (D.p == 4) run_kq<12, 2, FUSED, LM, XF>(D, lw, D.nwg, lds, best, keys);
            else if (D.p == 8) run_kq<12, 3, FUSED, LM, XF>(D, lw, D.nwg, lds, best, keys);
            else run_kq<12, 4, FUSED, LM, XF>(D, lw, D.nwg, lds, best, keys);
            break;
        case 13:
            if (D.p == 4) run_kq<13, 2, FUSED, LM, XF>(D, lw, D.nwg, lds, best, keys);
            else if (D.p == 8) run_kq<13, 3, FUSED, LM, XF>(D, lw, D.nwg, lds, best, keys);
            else run_kq<13, 4, FUSED, LM, XF>(D, lw, D.nwg, lds, best, keys);
            break;
        case 14:
            if (D.p == 4) run_kq<14, 2, FUSED, LM, XF>(D, lw, D.nwg, lds, best, keys);
            else if (D.p == 8) run_kq<14, 3, FUSED, LM, XF>(D, lw, D.nwg, lds, best, keys);
            else run_kq<14, 4, FUSED, LM, XF>(D, lw, D.nwg, lds, best, keys);
            break;
        default:
            if (D.p == 4 && D.nb == 32) run_q80r<32, FUSED, XF>(D, lw, D.nwg, lds, best, keys);
            else if (D.p == 4) run_q80r<16, FUSED, XF>(D, lw, D.nwg, lds, best, keys);
            else run_q80<FUSED, XF>(D, lw, D.nwg, lds, best, keys);
            break;
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
        lds_barrier();                                 // the logit stores need not complete first
        if (threadIdx.x == 0) {
            uint64_t m = wbest[0];
            for (int i = 1; i < 4; i++) m = wbest[i] > m ? wbest[i] : m;
            amax_partial[blockIdx.x] = m;
        }
    }
    // Top-k candidate and finished-block counters for the LM head's filter
    // kernel, which runs after this one on the same stream.
    if (zero_ctr && blockIdx.x == 0 && threadIdx.x < 2) zero_ctr[threadIdx.x] = 0;
}

void gemv_plan(GemvDesc &d) {
    if (d.type == 8) {
        d.nb = (int32_t)(d.k / QK8_0);
        // k = 512 / 1024: 4 rows per wave (p = 4); else one row per wave
        const bool rows4 = d.nb == 16 || d.nb == 32;
        d.p = rows4 ? 4 : 1;
        d.rows_per_tile = rows4 ? 16 : 4;
        d.lds_act = (d.nb * 36 + 15) & ~15;
    } else {
        d.nb = (int32_t)(d.k / QK_K);
        // groups per row: enough to cover the row in one step up to 16
        // super-blocks (k <= 4096), so a row costs one memory latency;
        // at least 4 (the kernel is instantiated for 4, 8 and 16)
        int p = 4;
        while (p < 16 && p < d.nb) p *= 2;
        d.p = p;
        d.rows_per_tile = 4 * (16 / p);
        // activations go straight to registers, or (fp32 row) through the
        // workgroup's quantized copy in LDS
        d.lds_act = d.xf32 ? d.nb * QXB : 0;
    }
    d.tr = d.rows_per_tile;
    d.tile_cap = 0;
    d.ntiles = (int32_t)((d.n + d.rows_per_tile - 1) / d.rows_per_tile);
    d.nwg = d.ntiles;
}

// Item offsets inside a matrix are 32-bit byte offsets.
int64_t gemv_max_matrix_bytes() { return (int64_t)0xffffffffLL; }

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
    // Descriptor starts are 16-bit fields: the grid stays below 2^16
    // workgroups (grid-stride covers the rest of a large matrix).
    const int cap = (0xffff / a.count < max_wg_per_desc) ? 0xffff / a.count : max_wg_per_desc;
    int32_t wg = 0, lds = 0;
    KArgs ka;
    uint32_t tab[8];
    for (int i = 0; i < 8; i++) tab[i] = 0xffffffffu;  // unused descriptors: first workgroup 0xffff
    for (int i = 0; i < a.count; i++) {
        GemvDesc &d = a.d[i];
        d.nwg = d.ntiles < cap ? d.ntiles : cap;
        d.wg0 = wg;
        wg += d.nwg;
        const int32_t need = d.lds_act + 4 * WBUF_BYTES;   // activation row | 4 wave windows
        lds = need > lds ? need : lds;
        KDesc &k = ka.d[i];
        k.w = d.w;
        k.xq = d.xq;
        k.y = d.y;
        k.n = (int32_t)d.n;
        k.type = d.type;
        k.nb = d.nb;
        k.p = d.p;
        k.rows_per_tile = d.rows_per_tile;
        k.ntiles = d.ntiles;
        k.nwg = d.nwg;
        k.lds_act = d.lds_act;
        k.wg0 = d.wg0;
        k.xf32 = d.xf32;
        const uint32_t sh = 16u * (uint32_t)(i & 1);
        tab[i >> 1] = (tab[i >> 1] & ~(0xffffu << sh)) | ((uint32_t)d.wg0 << sh);
    }
    a.lds_bytes = lds;
    if (grid_out) *grid_out = wg;
    // The LM head (argmax keys wanted) and streaming launches, whose waves
    // loop over many items, run the LM instantiation (two register sets in
    // turn); decode launches keep the leaner one.
    bool stream = amax_partial != nullptr;
    for (int i = 0; i < a.count; i++) stream = stream || a.d[i].ntiles > a.d[i].nwg;
    auto kern = stream ? (a.fused ? k_gemv<true, true, false> : k_gemv<false, true, false>)
                       : (a.fused ? k_gemv<true, false, false> : k_gemv<false, false, false>);
    if (a.d[0].xf32)                                   // fp32 rows (every descriptor of the launch)
        kern = stream ? (a.fused ? k_gemv<true, true, true> : k_gemv<false, true, true>)
                      : (a.fused ? k_gemv<true, false, true> : k_gemv<false, false, true>);
    hipLaunchKernelGGL(kern, dim3(wg), dim3(256), lds, s, tab[0], tab[1], tab[2], tab[3], tab[4], tab[5], tab[6],
                       tab[7], ka, amax_partial, zero_ctr);
    return hipGetLastError();
}

hipError_t launch_gemv(GemvArgs &a, int max_grid, hipStream_t s) {
    return launch_gemv_impl(a, max_grid, nullptr, nullptr, nullptr, s);
}

// ---- LM head: exact argmax and top-k -------------------------------------
// The GEMV leaves one key per workgroup: the maximum (value, -row) key of
// the rows it wrote. argmax = max over those keys.
//
// Top-k (keys compare by value, then lower row). The smallest of any k
// distinct logits is a lower bound on the k-th largest logit. The
// workgroup maxima are distinct logits, and so are the maxima of disjoint
// groups of G workgroups. k_topk_filter takes as its bound T the k-th
// largest group maximum, searched on the top 16 bits of the value key
// (low bits zero, so T stays a lower bound), and collects every logit
// whose value key is >= T: all of the top k are among them. The last
// filter block to finish ranks the candidates (topk_rank). If more than
// TOPK_CAND logits pass (a pathological flat distribution), it falls back
// to k exact passes over all logits.
#define TOPK_CAND 4096
// Workgroups of the LM-head GEMV (grid-stride over tiles), one maximum
// each: two per CU. Measured with argmax on 248320 x 1024: 1024 (four per
// CU) 40.7 us, 768 40.2, 512 39.6, 384 45.6, 256 48.9; counts that leave
// CUs unevenly loaded (640, 896) are slower than their neighbours.
#define LMHEAD_WG 512

__device__ __forceinline__ uint32_t valkey(float v) {
    uint32_t b = __float_as_uint(v);
    if (v == 0.0f) b = 0;
    return (v != v) ? 0u : ((b & 0x80000000u) ? ~b : (b | 0x80000000u));
}

__device__ __forceinline__ uint32_t dpp_mirror(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x140, 0xF, 0xF, true);   // row_mirror
}

// Largest T with zero low 16 bits such that at least k of the wave's keys
// are >= T (R keys per lane, read from keys[R * lane ...]): a bit-by-bit
// search from the top, one ballot per key and bit. T is wave-uniform.
template <int R>
__device__ uint32_t wave_bound(const uint32_t *keys, int k) {
    const int lane = threadIdx.x & 63;
    uint32_t x[R];
#pragma unroll
    for (int r = 0; r < R; r++) x[r] = keys[R * lane + r];
    uint32_t T = 0;
#pragma unroll
    for (int b = 31; b >= 16; b--) {
        const uint32_t c = T | (1u << b);
        int cnt = 0;
#pragma unroll
        for (int r = 0; r < R; r++) cnt += __popcll(__ballot(x[r] >= c));
        T = cnt >= k ? c : T;
    }
    return T;
}

// Sum of v over aligned groups of P lanes (P = 1, 2, 4, 8, 16), left in
// every lane of the group. All lanes must be active.
__device__ __forceinline__ int group_sum(int v, int P) {
    if (P >= 2) v += dpp_xor1(v);
    if (P >= 4) v += dpp_xor2(v);
    if (P >= 8) v += dpp_hmirror(v);
    if (P >= 16) v += (int)dpp_mirror((uint32_t)v);
    return v;
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
        for (int r = 0; r < R; r++) {
            // Lanes holding the same digit add together, one LDS atomic
            // per distinct digit of the wave: keys of similar logits share
            // their top digits, and same-address atomics serialize lane by
            // lane. After 4 rounds the rest add one by one.
            bool act = have[r] && (key[r] & mask) == prefix;
            const uint32_t dig = (uint32_t)(key[r] >> shift) & 255u;
            for (int it = 0; it < 4; it++) {
                const uint64_t pend = __ballot(act);
                if (pend == 0) break;
                const int leader = __builtin_ctzll(pend);
                const uint32_t d0 = (uint32_t)__builtin_amdgcn_readlane((int)dig, leader);
                const bool same = act && dig == d0;
                const uint64_t m = __ballot(same);
                if (lane == leader) atomicAdd(&hist[d0], (uint32_t)__builtin_popcountll(m));
                act = act && !same;
            }
            if (act) atomicAdd(&hist[dig], 1u);
        }
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

__device__ void topk_rank(const float *__restrict__ logits, int64_t n, const uint64_t *__restrict__ cand,
                          uint32_t c, int topk, int32_t *__restrict__ topk_idx, float *__restrict__ topk_val);

// Grid: ceil(n / 4096) blocks of 1024 when topk > 0, else one block.
// Block 0 writes the argmax. With topk > 0 every block finds the same
// bound T from the nparts (<= LMHEAD_WG) workgroup maxima, then collects
// its 4096 logits that reach it.
__global__ __launch_bounds__(1024) void k_topk_filter(const float *__restrict__ logits, int64_t n,
                                                      const uint64_t *__restrict__ partial, int nparts,
                                                      int topk, uint64_t *__restrict__ cand,
                                                      uint32_t *__restrict__ ctr, int32_t *__restrict__ argmax,
                                                      int32_t *__restrict__ topk_idx,
                                                      float *__restrict__ topk_val) {
    __shared__ uint32_t gkey[1024];                    // group maxima (value keys)
    __shared__ uint64_t red[16];
    __shared__ uint32_t tsh;
    const int t = threadIdx.x, lane = t & 63;
    const uint64_t pk = t < nparts ? partial[t] : 0;
    const int64_t base = (int64_t)blockIdx.x * 4096;
    float v[4];
#pragma unroll
    for (int r = 0; r < 4; r++) {
        const int64_t i = base + t + 1024 * r;
        v[r] = (topk > 0 && i < n) ? logits[i] : 0.0f;
    }
    float l0 = 0.0f;
    if (blockIdx.x == 0 && t == 64) l0 = logits[0];
    // Group size: the largest of 16, 4, 1 that leaves at least k groups;
    // G = 0: fewer maxima than k (a tiny vocabulary), every logit passes.
    const int G = (nparts + 15) / 16 >= topk ? 16 : (nparts + 3) / 4 >= topk ? 4 : nparts >= topk ? 1 : 0;
    if (topk > 0 && G > 0) {
        uint32_t m = (uint32_t)(pk >> 32);
        if (G >= 4) {
            m = max(m, (uint32_t)dpp_xor1((int)m));
            m = max(m, (uint32_t)dpp_xor2((int)m));
        }
        if (G >= 16) {
            m = max(m, (uint32_t)dpp_hmirror((int)m));
            m = max(m, dpp_mirror(m));
        }
        if ((lane & (G - 1)) == 0) gkey[t / G] = m;
    }
    if (blockIdx.x == 0) {
        uint64_t m = pk;
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) {
            const uint32_t lo = __shfl_xor((uint32_t)m, off), hi = __shfl_xor((uint32_t)(m >> 32), off);
            const uint64_t o = ((uint64_t)hi << 32) | lo;
            m = o > m ? o : m;
        }
        if (lane == 0) red[t >> 6] = m;
    }
    __syncthreads();
    if (blockIdx.x == 0 && t == 64) {                  // wave 1; wave 0 searches T
        uint64_t b = red[0];
        for (int i = 1; i < 16; i++) b = red[i] > b ? red[i] : b;
        int32_t best = (int32_t)(0xffffffffu - (uint32_t)(b & 0xffffffffu));
        if (l0 != l0) best = 0;                        // sample_argmax: v[0] = NaN never loses
        *argmax = best;
    }
    if (topk <= 0) return;                             // uniform
    if (t < 64) {
        uint32_t T = 0;
        if (G == 16) T = wave_bound<1>(gkey, topk);
        else if (G == 4) T = wave_bound<4>(gkey, topk);
        else if (G == 1) T = wave_bound<16>(gkey, topk);
        if (t == 0) tsh = T;
    }
    __syncthreads();
    const uint32_t T = tsh;
#pragma unroll
    for (int r = 0; r < 4; r++) {
        const int64_t i = base + t + 1024 * r;
        if (i < n && valkey(v[r]) >= T) {
            const uint32_t slot = atomicAdd(ctr, 1u);
            if (slot < TOPK_CAND)
                __hip_atomic_exchange(&cand[slot], ((uint64_t)valkey(v[r]) << 32) | (0xffffffffu - (uint32_t)i),
                                      __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    // The last block to finish ranks the candidates: every thread's
    // atomics have completed (waitcnt) before the block counts itself done.
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (t == 0) {
        const uint32_t done = __hip_atomic_fetch_add(&ctr[1], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        tsh = done == gridDim.x - 1;
    }
    __syncthreads();
    if (!tsh) return;                                  // uniform
    const uint32_t c = __hip_atomic_load(&ctr[0], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    topk_rank(logits, n, cand, c, topk, topk_idx, topk_val);
}

// The exact top-k of the filtered candidates, ranked value-descending /
// row-ascending, by the filter's last block (all 1024 threads). The
// candidates and their count were written by atomics at agent scope, which
// bypass the per-XCD L2, so plain agent-scope atomic loads see them.
//
// NaN follows topk_collect (slm/sampler.c:70-93): its first k rows fill the
// slots, and a NaN slot never compares as the worst one, so it is never
// replaced; a NaN after the fill never enters (NaN > x is false). With row
// 0 NaN the worst slot stays 0 and nothing is ever replaced: the set is
// rows 0..k-1. Otherwise the set is the c NaN rows among 1..k-1 plus the
// k - c largest numbers. Ranked here: numbers value-descending, then the
// NaN rows by row.
__device__ __forceinline__ uint64_t agent_load(const uint64_t *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ void topk_rank(const float *__restrict__ logits, int64_t n, const uint64_t *__restrict__ cand,
                          uint32_t c, int topk, int32_t *__restrict__ topk_idx, float *__restrict__ topk_val) {
    __shared__ uint32_t hist[258];
    __shared__ uint64_t win[1024];                     // candidates (ranking) or winners
    __shared__ uint64_t red[16];
    __shared__ uint32_t nwin, nnan, frozen;
    __shared__ uint8_t nanrow[QK_TOPK_MAX_DEV];        // NaN among the first k rows
    const int t = threadIdx.x;
    const uint64_t mine = agent_load(&cand[t]);        // t < 1024 <= TOPK_CAND; used when t < c
    const float fill = t < topk && t < n ? logits[t] : 0.0f;
    const bool fnan = t < topk && t < n && fill != fill;
    if (t == 0) {
        nwin = 0;
        nnan = 0;
        frozen = fnan;
    }
    if (t < topk) nanrow[t] = fnan;
    __syncthreads();
    if (fnan && t > 0) atomicAdd(&nnan, 1u);
    __syncthreads();
    // numbers to rank: all k when row 0 is NaN (the fill itself is ranked),
    // else k minus the NaN rows of the fill
    const int kk = frozen ? topk : topk - (int)nnan;
    int nw;                                            // keys in win[] to rank
    if (frozen) {
        if (t < topk) win[t] = ((uint64_t)valkey(fill) << 32) | (0xffffffffu - (uint32_t)t);
        nw = topk;
    } else if (c <= 1024) {
        // Few candidates: rank every number among them directly.
        if (t < (int)c && (mine >> 32) != 0) win[atomicAdd(&nwin, 1u)] = mine;
        __syncthreads();
        nw = (int)nwin;
    } else if (c <= TOPK_CAND) {
        uint64_t key[4];
        bool have[4];
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const uint32_t i = t + 1024 * r;
            key[r] = r == 0 ? mine : i < c ? agent_load(&cand[i]) : 0;
            have[r] = i < c && (key[r] >> 32) != 0;    // value key 0: NaN
        }
        const uint64_t T = block_kth_largest<4, 64, uint64_t>(key, have, kk, hist);
#pragma unroll
        for (int r = 0; r < 4; r++)
            if (have[r] && key[r] >= T) win[atomicAdd(&nwin, 1u)] = key[r];
        nw = kk;
    } else {
        // Fallback: k exact passes, each taking the largest key below the
        // previous winner (NaN keys, 0, never win).
        uint64_t prev = ~(uint64_t)0;
        for (int r = 0; r < kk; r++) {
            uint64_t b = 0;
            for (int64_t i = t; i < n; i += 1024) {
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
            if ((t & 63) == 0) red[t >> 6] = b;
            __syncthreads();
            uint64_t bb = red[0];
            for (int i = 1; i < 16; i++) bb = red[i] > bb ? red[i] : bb;
            if (t == 0) win[r] = bb;
            prev = bb;
        }
        nw = kk;
    }
    __syncthreads();
    // Rank the keys (all distinct): P lanes per key, lane j of a group
    // counts the keys j, j + P, ... above its key; the group's lane 0
    // writes the key at its rank when that is below k.
    const int P = nw <= 64 ? 16 : nw <= 128 ? 8 : nw <= 256 ? 4 : nw <= 512 ? 2 : 1;
    const int i = t / P, j = t % P;
    const bool live = i < nw;
    const uint64_t me = live ? win[i] : 0;
    const int32_t idx = (int32_t)(0xffffffffu - (uint32_t)(me & 0xffffffffu));
    float val = 0.0f;
    if (live && j == 0) val = logits[idx];             // in flight during the count
    int cnt = 0;
    if (live)
        for (int q = j; q < nw; q += P) cnt += win[q] > me;
    cnt = group_sum(cnt, P);
    if (live && j == 0 && cnt < kk) {
        topk_idx[cnt] = idx;
        topk_val[cnt] = val;
    }
    // the fill's NaN rows after the numbers, by row
    if (!frozen && fnan && t > 0) {
        int below = 0;
        for (int u = 1; u < t; u++) below += nanrow[u];
        topk_idx[kk + below] = t;
        topk_val[kk + below] = fill;
    }
}

static int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

size_t lmhead_cand_bytes(int64_t, int) {
    // argmax partials (<= LMHEAD_WG workgroups) | candidate keys | counter
    return (size_t)(LMHEAD_WG + TOPK_CAND) * sizeof(uint64_t) + 64;
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
    uint64_t *cand = partial + LMHEAD_WG;
    uint32_t *ctr = reinterpret_cast<uint32_t *>(cand + TOPK_CAND);
    int grid = 0;
    hipError_t e = launch_gemv_impl(a, LMHEAD_WG, partial, ctr, &grid, s);
    if (e != hipSuccess) return e;
    if (grid > LMHEAD_WG) return hipErrorInvalidValue;
    const unsigned fgrid = topk > 0 ? (unsigned)cdiv(n, 4096) : 1u;
    hipLaunchKernelGGL(k_topk_filter, dim3(fgrid), dim3(1024), 0, s, logits, n, partial, grid, topk, cand, ctr,
                       argmax, topk_idx, topk_val);
    return hipGetLastError();
}

}  // namespace qk
