// qk_gemm.hip -- chunked-prefill GEMM over native GGUF K-quant and Q8_0
// blocks (gfx950, int8 MFMA). The K-quant kernel is described here; its
// 128-token-tile form for long prompts (k_gemm_w) and the Q8_0 kernel
// (k_gemm_q80) have their own descriptions further down.
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
// Work decomposition: a 512-thread workgroup owns a 64-token x BN-row
// output tile (BN = 64, or 32 when 64-row tiles would leave CUs idle) and
// walks the super-blocks of K in order. For each one it stages the 64
// activation rows (int8 Q8_K quants, scale, bsum pairs; threads 0-255)
// and the BN weight rows, dequantised to int8 with their sub-block
// scales (the next 4*BN threads), into LDS; the next super-block's raw
// bytes are loaded into registers meanwhile. Each 32x32 sub-tile is
// computed by KS = 128 / BN waves, each over 1/KS of the super-block's k
// range (integer sums: exact in any order); the waves of a sub-tile
// exchange their int32 parts through LDS and each finishes 16/KS of the
// 16 outputs per lane:
//
//  * Q4_K / Q5_K: the 6-bit sub-block scales are split into two 3-bit
//    digits and baked into int8 weight planes (plus a 5th-bit plane for
//    Q5_K), so one chain of v_mfma_i32_32x32x32_i8 per plane accumulates
//    the wave's part of the super-block and
//    isum = acc0 + 8*acc1 (+ 16*acc2); mins from the Q8_K bsums
//    (simd/quants.h:283-304, 324-349);
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

#include <type_traits>

namespace qk {

typedef int32_t v4i __attribute__((ext_vector_type(4)));
typedef int32_t v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));

#define GM_BM 64                      // tokens per workgroup tile
#define GM_LD 272                     // LDS row stride of the int8 tiles (256 + 16)

// Dequantised weight planes per super-block. Q4_K / Q5_K: the 6-bit
// sub-block scale sc = 8*hi + lo is split into two 3-bit digits and baked
// into the weights, plane 0 = q4 * lo, plane 1 = q4 * hi (<= 105, int8);
// Q5_K adds plane 2 = (5th bit) * sc (<= 63). One MFMA chain per plane
// then accumulates a whole super-block, and
//   isum = acc0 + 8*acc1 (+ 16*acc2)
// exactly (every int8 product and every int32 sum is exact). Q6_K: one
// plane, u6 - 32 in [-32, 31], scaled per 16-element sub-block after each
// MFMA.
template <int TYPE> struct Planes { static constexpr int n = TYPE == 12 ? 2 : (TYPE == 13 ? 3 : 1); };

template <int NP, int BN>
struct __attribute__((aligned(16))) GemmLds {
    int8_t a[GM_BM][GM_LD];           // activation quants of the super-block
    int8_t b[NP][BN][GM_LD];          // dequantised int8 weight planes
    int8_t am[GM_BM][16];             // bsum pairs p = 128*hi + lo: lo[8] (0..127) | hi[8] (-64..63)
    float yd[GM_BM];                  // Q8_K d per token
    int8_t sc[BN][16];                // Q6_K sub-block scales per weight row
    uint8_t mn[BN][8];                // 6-bit mins (Q4_K / Q5_K)
    float wd[BN];                     // fp16 d, widened
    float wdm[BN];                    // fp16 dmin, widened
};

__device__ __forceinline__ void lds_st16(void *p, uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
    *(QK_LDS uint4 *)p = make_uint4(a, b, c, d);
}

// ---- staging ---------------------------------------------------------------
// Each super-block step moves its raw bytes in two halves: load_*() issues
// every global load of the step into registers, and store_*() unpacks
// those registers into LDS; the kernel loads step i+1 while it computes
// step i. Thread tid works on token / weight row tid/4 and quarter
// q = tid%4 of it, so all of a thread's loads in a step are immediate
// offsets from one row pointer computed once per kernel.

// Activations: quarter q of a token holds qs[64q, 64q+64) of its 292-byte
// Q8_K block (d | qs[256] | bsums[16]) as four 16-byte loads at 4-byte
// aligned offsets, bsum pairs 2q and 2q+1, and d. The buffer covers the
// workgroup's tokens, so rows past m read zeros.
struct ActRaw { uint4 q[4]; uint32_t b0, b1, d; };

__device__ __forceinline__ void load_act(ActRaw &a, __amdgpu_buffer_rsrc_t r, int row_off, int q, int i) {
    const int o = row_off + i * Q8K_BYTES;
#pragma unroll
    for (int j = 0; j < 4; j++) a.q[j] = bl128(r, o + 4 + 64 * q + 16 * j);
    a.b0 = bl32(r, o + 260 + 8 * q);
    a.b1 = bl32(r, o + 264 + 8 * q);
    a.d = bl32(r, o);
}

// bsum pair j (bsums[2j] + bsums[2j+1], one dword of the block) as two
// int8 digits of the mins operand.
template <typename GL>
__device__ __forceinline__ void store_pair(GL &s, int t, int j, uint32_t v) {
    const int32_t p = (int32_t)(int16_t)(v & 0xffffu) + (int32_t)(int16_t)(v >> 16);
    s.am[t][j] = (int8_t)(p & 127);
    s.am[t][8 + j] = (int8_t)(p >> 7);
}

template <typename GL>
__device__ __forceinline__ void store_act(GL &s, const ActRaw &a, int t, int q) {
#pragma unroll
    for (int j = 0; j < 4; j++) *(QK_LDS uint4 *)&s.a[t][64 * q + 16 * j] = a.q[j];   // rows: 16-byte aligned
    store_pair(s, t, 2 * q, a.b0);
    store_pair(s, t, 2 * q + 1, a.b1);
    if (q == 0) s.yd[t] = __uint_as_float(a.d);
}

// Mins, d and dmin of a Q4_K / Q5_K header (d | dmin | scales[12]).
template <typename GL>
__device__ __forceinline__ void store_kq_header(GL &s, int r, const uint4 v) {
    int32_t sc, mm;
#pragma unroll
    for (int j = 0; j < 8; j++) {
        scale_min(v.y, v.z, v.w, j, sc, mm);
        s.mn[r][j] = (uint8_t)mm;
    }
    s.wd[r] = h2f(v.x & 0xffffu);
    s.wdm[r] = h2f(v.x >> 16);
}

// Bytes of x times d, byte by byte, for products below 256: two packed
// 16-bit multiplies (each 16-bit lane holds two bytes b0 + 256*b1; with
// b*d < 256 the low byte's product never carries into the high byte's).
__device__ __forceinline__ uint32_t bmul(uint32_t x, uint32_t d) {
    typedef unsigned short us2 __attribute__((ext_vector_type(2)));
    const us2 a = __builtin_bit_cast(us2, x);
    const us2 b = {(unsigned short)d, (unsigned short)d};
    return __builtin_bit_cast(uint32_t, a * b);
}

__device__ __forceinline__ void st16(int8_t *p, const uint32_t (&v)[4]) {
    *(QK_LDS uint4 *)p = make_uint4(v[0], v[1], v[2], v[3]);
}

// 16 four-bit weights (one 16-byte run of nibble bytes, values 0..15) of
// sub-block `sb` at element offset e, times the two digits of its scale.
template <typename GL>
__device__ __forceinline__ void store_q4_digits(GL &s, int r, int e, const uint32_t (&q)[4], int32_t sc) {
    const uint32_t lo = (uint32_t)sc & 7u, hi = (uint32_t)sc >> 3;
    uint32_t a[4], b[4];
#pragma unroll
    for (int k = 0; k < 4; k++) {
        a[k] = bmul(q[k], lo);
        b[k] = bmul(q[k], hi);
    }
    st16(&s.b[0][r][e], a);
    st16(&s.b[1][r][e], b);
}

// Q4_K (144 B): header | qs[128]; qs[32c + l] low nibble is element
// 64c + l (sub-block 2c), high nibble 64c + 32 + l (sub-block 2c+1).
// Quarter q takes the 16-byte qs pieces q and q+4 (chunk c = q/2 and
// 2 + q/2, positions 16(q&1)..+16) and needs the header for their scales.
struct WRaw12 { uint4 hdr, p0, p1; };

__device__ __forceinline__ void load_w(WRaw12 &a, const uint8_t *row, int q, int i) {
    a.hdr = a.p0 = a.p1 = make_uint4(0, 0, 0, 0);
    if (!row) return;
    const uint8_t *p = row + (int64_t)i * Q4K_BYTES;
    a.hdr = ld16(p);
    a.p0 = ld16(p + 16 + 16 * q);
    a.p1 = ld16(p + 80 + 16 * q);
}

template <typename GL>
__device__ __forceinline__ void store_piece4(GL &s, int r, int c, int l0, const uint4 v, const uint4 hdr) {
    const uint32_t M = 0x0F0F0F0Fu;
    const uint32_t lo[4] = {v.x & M, v.y & M, v.z & M, v.w & M};
    const uint32_t hi[4] = {(v.x >> 4) & M, (v.y >> 4) & M, (v.z >> 4) & M, (v.w >> 4) & M};
    int32_t sc0, m0, sc1, m1;
    scale_min(hdr.y, hdr.z, hdr.w, 2 * c, sc0, m0);
    scale_min(hdr.y, hdr.z, hdr.w, 2 * c + 1, sc1, m1);
    store_q4_digits(s, r, 64 * c + l0, lo, sc0);
    store_q4_digits(s, r, 64 * c + 32 + l0, hi, sc1);
}

template <typename GL>
__device__ __forceinline__ void store_w(GL &s, const WRaw12 &a, int r, int q) {
    if (q == 0) store_kq_header(s, r, a.hdr);
    store_piece4(s, r, q >> 1, 16 * (q & 1), a.p0, a.hdr);
    store_piece4(s, r, 2 + (q >> 1), 16 * (q & 1), a.p1, a.hdr);
}

// Q5_K (176 B): header | qh[32] | qs[128]. Element 64c + l gets bit 2c of
// qh[l] as its 5th bit, element 64c + 32 + l bit 2c+1; quarter q needs the
// qh bytes of its positions 16(q&1)..+16. Planes 0/1 carry the low four
// bits times the scale digits, plane 2 the 5th bit times the scale.
struct WRaw13 { uint4 hdr, p0, p1, qh; };

__device__ __forceinline__ void load_w(WRaw13 &a, const uint8_t *row, int q, int i) {
    a.hdr = a.p0 = a.p1 = a.qh = make_uint4(0, 0, 0, 0);
    if (!row) return;
    const uint8_t *p = row + (int64_t)i * Q5K_BYTES;
    a.hdr = ld16(p);
    a.qh = ld16(p + 16 + 16 * (q & 1));
    a.p0 = ld16(p + 48 + 16 * q);
    a.p1 = ld16(p + 112 + 16 * q);
}

template <typename GL>
__device__ __forceinline__ void store_piece5(GL &s, int r, int c, int l0, const uint4 v, const uint4 h,
                                             const uint4 hdr) {
    const uint32_t M = 0x0F0F0F0Fu, B1 = 0x01010101u;
    const uint32_t s0 = 2 * c, s1 = 2 * c + 1;
    const uint32_t lo[4] = {v.x & M, v.y & M, v.z & M, v.w & M};
    const uint32_t hi[4] = {(v.x >> 4) & M, (v.y >> 4) & M, (v.z >> 4) & M, (v.w >> 4) & M};
    const uint32_t hl[4] = {(h.x >> s0) & B1, (h.y >> s0) & B1, (h.z >> s0) & B1, (h.w >> s0) & B1};
    const uint32_t hh[4] = {(h.x >> s1) & B1, (h.y >> s1) & B1, (h.z >> s1) & B1, (h.w >> s1) & B1};
    int32_t sc0, m0, sc1, m1;
    scale_min(hdr.y, hdr.z, hdr.w, 2 * c, sc0, m0);
    scale_min(hdr.y, hdr.z, hdr.w, 2 * c + 1, sc1, m1);
    store_q4_digits(s, r, 64 * c + l0, lo, sc0);
    store_q4_digits(s, r, 64 * c + 32 + l0, hi, sc1);
    uint32_t a[4], b[4];
#pragma unroll
    for (int k = 0; k < 4; k++) {
        a[k] = bmul(hl[k], (uint32_t)sc0);
        b[k] = bmul(hh[k], (uint32_t)sc1);
    }
    st16(&s.b[2][r][64 * c + l0], a);
    st16(&s.b[2][r][64 * c + 32 + l0], b);
}

template <typename GL>
__device__ __forceinline__ void store_w(GL &s, const WRaw13 &a, int r, int q) {
    if (q == 0) store_kq_header(s, r, a.hdr);
    store_piece5(s, r, q >> 1, 16 * (q & 1), a.p0, a.qh, a.hdr);
    store_piece5(s, r, 2 + (q >> 1), 16 * (q & 1), a.p1, a.qh, a.hdr);
}

// Four bytes u6 in [0, 63] -> four int8 bytes u6 - 32. u6 ^ 0x20 is
// u6 - 32 as a 6-bit two's-complement number (bit 5 the sign); copying
// bit 5 into bits 6 and 7 sign-extends it to 8 bits, byte by byte.
__device__ __forceinline__ uint32_t u6_minus_32(uint32_t x) {
    const uint32_t v = x ^ 0x20202020u;
    const uint32_t sg = v & 0x20202020u;
    return v | (sg << 1) | (sg << 2);
}

// Q6_K (210 B, 2-byte aligned): element 128h + 32qq + l (l < 32) is
// ql[64h + l + 32(qq&1)] (low nibble for qq < 2, high for qq >= 2) | the
// 2 bits of qh[32h + l] at 2qq, minus 32. Quarter q covers positions
// l0..l0+15 (l0 = 16(q&1)) of all four quarters of half h = q/2, read as
// three 16-byte runs, each through the five aligned dwords that contain
// it (a 16-byte and a 4-byte load; the last ends at most at byte 196 of
// the block); quarter 0 also reads the 16 scale bytes the same way and d.
// The buffer starts at the 4-byte aligned address at or below the tile's
// first row and ends with its last row, so offsets are 32-bit and every
// byte a lane uses lies inside it. Rows past n read zeros, and so does the
// unused fifth scale dword of the tile's last block when sh = 0.
struct WRaw14 { uint32_t v[15]; uint4 sc; uint32_t sc4, d, sh; };

__device__ __forceinline__ void load_w(WRaw14 &a, __amdgpu_buffer_rsrc_t r, int row_off, int q, int i) {
    const int b = row_off + i * Q6K_BYTES;             // block start; the base is 4-byte aligned
    const int h = q >> 1, l0 = 16 * (q & 1);
    const int sh = b & 3;
    a.sh = (uint32_t)sh;
    const int p0 = b - sh + 64 * h + l0, p2 = b - sh + 128 + 32 * h + l0;
    const uint4 x0 = bl128(r, p0), x1 = bl128(r, p0 + 32), x2 = bl128(r, p2);
    a.v[0] = x0.x, a.v[1] = x0.y, a.v[2] = x0.z, a.v[3] = x0.w, a.v[4] = bl32(r, p0 + 16);
    a.v[5] = x1.x, a.v[6] = x1.y, a.v[7] = x1.z, a.v[8] = x1.w, a.v[9] = bl32(r, p0 + 48);
    a.v[10] = x2.x, a.v[11] = x2.y, a.v[12] = x2.z, a.v[13] = x2.w, a.v[14] = bl32(r, p2 + 16);
    // every quarter loads them (one wave-wide load each); quarter 0 stores them
    a.sc = bl128(r, b - sh + 192);
    a.sc4 = bl32(r, b - sh + 208);                     // needed only when sh > 0, then inside the block
    a.d = __builtin_amdgcn_raw_buffer_load_b16(r, b + 208, 0, 0);
}

// The same registers from plain loads (64-row tiles, where the wider loads
// above push the kernel past its register budget). The fifth scale dword
// is read only when sh > 0, so no load passes the block's end.
__device__ __forceinline__ void load_w(WRaw14 &a, const uint8_t *row, int q, int i) {
#pragma unroll
    for (int j = 0; j < 15; j++) a.v[j] = 0;
    a.sc = make_uint4(0, 0, 0, 0);
    a.sc4 = a.d = a.sh = 0;
    if (!row) return;
    const uint8_t *blk = row + (int64_t)i * Q6K_BYTES;
    const int h = q >> 1, l0 = 16 * (q & 1);
    const uint32_t sh = (uint32_t)reinterpret_cast<uintptr_t>(blk) & 3u;
    a.sh = sh;
    const uint8_t *p0 = blk - sh + 64 * h + l0, *p2 = blk - sh + 128 + 32 * h + l0;
#pragma unroll
    for (int j = 0; j < 5; j++) {
        a.v[j] = ld32(p0 + 4 * j);
        a.v[5 + j] = ld32(p0 + 32 + 4 * j);
        a.v[10 + j] = ld32(p2 + 4 * j);
    }
    if (q == 0) {
        const uint8_t *ps = blk - sh + 192;
        a.sc = make_uint4(ld32(ps), ld32(ps + 4), ld32(ps + 8), ld32(ps + 12));
        if (sh) a.sc4 = ld32(ps + 16);
        a.d = ld_u16(blk + 208);
    }
}

template <typename GL>
__device__ __forceinline__ void store_w(GL &s, const WRaw14 &a, int r, int q) {
    const uint32_t sh = a.sh;
    if (q == 0) {
        *(QK_LDS uint4 *)&s.sc[r][0] = make_uint4(__builtin_amdgcn_alignbyte(a.sc.y, a.sc.x, sh),
                                                  __builtin_amdgcn_alignbyte(a.sc.z, a.sc.y, sh),
                                                  __builtin_amdgcn_alignbyte(a.sc.w, a.sc.z, sh),
                                                  __builtin_amdgcn_alignbyte(a.sc4, a.sc.w, sh));
        s.wd[r] = h2f(a.d);
    }
    const int h = q >> 1, l0 = 16 * (q & 1);
    uint32_t qa[4], qb[4], hh[4];
#pragma unroll
    for (int k = 0; k < 4; k++) {
        qa[k] = __builtin_amdgcn_alignbyte(a.v[k + 1], a.v[k], sh);       // quarters 0 / 2
        qb[k] = __builtin_amdgcn_alignbyte(a.v[k + 6], a.v[k + 5], sh);   // quarters 1 / 3
        hh[k] = __builtin_amdgcn_alignbyte(a.v[k + 11], a.v[k + 10], sh);
    }
    const uint32_t M = 0x0F0F0F0Fu, T = 0x30303030u;
    uint32_t o0[4], o1[4], o2[4], o3[4];
#pragma unroll
    for (int k = 0; k < 4; k++) {
        o0[k] = u6_minus_32((qa[k] & M) | ((hh[k] << 4) & T));
        o1[k] = u6_minus_32((qb[k] & M) | ((hh[k] << 2) & T));
        o2[k] = u6_minus_32(((qa[k] >> 4) & M) | (hh[k] & T));
        o3[k] = u6_minus_32(((qb[k] >> 4) & M) | ((hh[k] >> 2) & T));
    }
    lds_st16(&s.b[0][r][128 * h + l0], o0[0], o0[1], o0[2], o0[3]);
    lds_st16(&s.b[0][r][128 * h + 32 + l0], o1[0], o1[1], o1[2], o1[3]);
    lds_st16(&s.b[0][r][128 * h + 64 + l0], o2[0], o2[1], o2[2], o2[3]);
    lds_st16(&s.b[0][r][128 * h + 96 + l0], o3[0], o3[1], o3[2], o3[3]);
}

// Workgroup barrier over LDS only: it waits for this thread's LDS
// accesses, not for global loads in flight, so the next super-block's
// loads stay outstanding across it.
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

template <int TYPE> struct WRawOf;
template <> struct WRawOf<12> { typedef WRaw12 T; };
template <> struct WRawOf<13> { typedef WRaw13 T; };
template <> struct WRawOf<14> { typedef WRaw14 T; };

// Output element v (0..15) of a lane in a 32x32 MFMA tile: column (weight
// row) = lane % 32, row (token) = 8*(v/4) + 4*(lane/32) + v%4.
__device__ __forceinline__ int tok_of(int v, int h) { return 8 * (v >> 2) + 4 * h + (v & 3); }

struct NoRaw {};

// BN = 64: four 32x32 sub-tiles, two waves each (halves of the super-
// block's k); BN = 32: two sub-tiles, four waves each (quarters). Either
// way 8 waves; each wave finishes VPW = 16 / KS of its sub-tile's 16
// outputs per lane after the exchange.
template <int TYPE, bool FUSED, int BN>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(4)))
void k_gemm(const uint8_t *__restrict__ w, int64_t n, int nb, const uint8_t *__restrict__ xq, int64_t m,
            float *__restrict__ y) {
    constexpr int BB = TYPE == 12 ? Q4K_BYTES : (TYPE == 13 ? Q5K_BYTES : Q6K_BYTES);
    constexpr int NT = BN / 32;                              // sub-tile columns
    constexpr int NSUB = 2 * NT;                             // sub-tiles
    constexpr int KS = 8 / NSUB;                             // waves per sub-tile
    constexpr int VPW = 16 / KS;                             // outputs per lane a wave finishes
    constexpr bool ALIAS = TYPE == 13 && BN == 64;           // Q5_K: exchange through the activation tile
    constexpr int XCH = NSUB * KS * (KS - 1) * VPW * 64;     // exchange words
    __shared__ GemmLds<Planes<TYPE>::n, BN> s;
    __shared__ int32_t xch_mem[ALIAS ? 1 : XCH];
    int32_t *xch = ALIAS ? reinterpret_cast<int32_t *>(&s.a[0][0]) : xch_mem;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int col = lane & 31, h = lane >> 5;
    const int sub = wave % NSUB, g = wave / NSUB;            // sub-tile, part of the super-block's k
    const int tm = 32 * (sub / NT), tn = 32 * (sub % NT);
    const int64_t r0 = (int64_t)blockIdx.x * BN, t0 = (int64_t)blockIdx.y * GM_BM;
    // staging roles: threads 0..255 stage activation rows, the next 4*BN
    // weight rows, the rest (BN = 32) nothing; row st of the tile, quarter sq
    const int role = threadIdx.x < 256 ? 0 : (threadIdx.x < 256 + 4 * BN ? 1 : 2);
    const int st = (threadIdx.x & 255) >> 2, sq = threadIdx.x & 3;
    // activation rows of this token tile: one buffer of at most 64 x 64 x
    // 292 bytes, so every offset is 32-bit
    const int mrows = (m - t0 < GM_BM) ? (int)(m - t0) : GM_BM;
    const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t *>(xq + t0 * nb * Q8K_BYTES), 0, mrows * nb * Q8K_BYTES, 0x00020000);
    const int xoff = st * nb * Q8K_BYTES;
    const uint8_t *wrow = (role == 1 && r0 + st < n) ? w + (r0 + st) * nb * BB : nullptr;
    // Q6_K weight rows of this tile as one buffer (see load_w)
    const uint8_t *wtile = w + r0 * nb * BB;
    const int wmis = (int)(reinterpret_cast<uintptr_t>(wtile) & 3u);
    const int nrows = (n - r0 < BN) ? (int)(n - r0) : BN;
    const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t *>(wtile - wmis), 0, wmis + nrows * nb * BB, 0x00020000);
    const int woff = wmis + st * nb * BB;

    const int8_t *arow = &s.a[tm + col][0];
    const v16i zero = {0};
    // The loop runs in one copy per staging role, so that a thread holds
    // registers for its own raw bytes only.
    auto body = [&](auto &raw, auto role_c) {
        constexpr int R = decltype(role_c)::value;
        float sum[VPW];
#pragma unroll
        for (int v = 0; v < VPW; v++) sum[v] = 0.0f;
        if constexpr (R == 1) {
            if constexpr (TYPE == 14 && BN == 32) load_w(raw, wr, woff, sq, 0);
            else load_w(raw, wrow, sq, 0);
        }
        if constexpr (R == 0) load_act(raw, xr, xoff, sq, 0);

        for (int i = 0; i < nb; i++) {
            lds_barrier();                                       // previous super-block's reads done
            if constexpr (R == 1) store_w(s, raw, st, sq);
            if constexpr (R == 0) store_act(s, raw, st, sq);
            if (i + 1 < nb) {                                    // next super-block in flight during compute
                if constexpr (R == 1) {
                    if constexpr (TYPE == 14 && BN == 32) load_w(raw, wr, woff, sq, i + 1);
                    else load_w(raw, wrow, sq, i + 1);
                }
                if constexpr (R == 0) load_act(raw, xr, xoff, sq, i + 1);
            }
            lds_barrier();

            // this wave's part of the super-block's k range
            int32_t isum[16];
            if constexpr (TYPE == 14) {
                // per 16-element sub-block: MFMA, then times its int8 scale
                constexpr int SPW = 16 / KS;
                const int8_t *brow = &s.b[0][tn + col][0];
#pragma unroll
                for (int v = 0; v < 16; v++) isum[v] = 0;
                uint32_t scw[SPW / 4];
#pragma unroll
                for (int q = 0; q < SPW / 4; q++) scw[q] = *(const QK_LDS uint32_t *)&s.sc[tn + col][SPW * g + 4 * q];
#pragma unroll
                for (int j = 0; j < SPW; j++) {
                    const int sb = SPW * g + j;
                    const long av = *(const QK_LDS long *)(arow + 16 * sb + 8 * h);
                    const long bv = *(const QK_LDS long *)(brow + 16 * sb + 8 * h);
                    const v16i d = __builtin_amdgcn_mfma_i32_32x32x16_i8(av, bv, zero, 0, 0, 0);
                    const int32_t scv = (int32_t)(int8_t)(scw[j >> 2] >> (8 * (j & 3)));
#pragma unroll
                    for (int v = 0; v < 16; v++) isum[v] += __mul24(scv, d[v]);
                }
            } else {
                // one accumulation chain per digit plane over the part
                constexpr int NP = Planes<TYPE>::n;
                constexpr int CPW = 8 / KS;
                v16i acc[NP];
#pragma unroll
                for (int pl = 0; pl < NP; pl++) acc[pl] = zero;
#pragma unroll
                for (int j = 0; j < CPW; j++) {
                    const int c = CPW * g + j;
                    const v4i av = *(const QK_LDS v4i *)(arow + 32 * c + 16 * h);
#pragma unroll
                    for (int pl = 0; pl < NP; pl++) {
                        const v4i bv = *(const QK_LDS v4i *)(&s.b[pl][tn + col][32 * c + 16 * h]);
                        acc[pl] = __builtin_amdgcn_mfma_i32_32x32x32_i8(av, bv, acc[pl], 0, 0, 0);
                    }
                }
#pragma unroll
                for (int v = 0; v < 16; v++) {
                    int32_t t = acc[0][v] + 8 * acc[1][v];
                    if constexpr (NP == 3) t += 16 * acc[2][v];
                    isum[v] = t;
                }
            }
            if constexpr (KS == 4) {
                // Four parts: one copy of the rest of the step per part, so
                // every part index is a compile-time constant (the runtime
                // selects below cost 2.5-4 % here; with two parts a copy per
                // part gains nothing, and for 64-row Q6_K tiles it exceeds the
                // register budget).
                auto finish = [&](auto gc) __attribute__((always_inline)) {
                    constexpr int G = decltype(gc)::value;
                    if (ALIAS) lds_barrier();                            // every wave is done reading s.a
#pragma unroll
                    for (int o = 0; o < KS; o++) {
                        if (o == G) continue;
                        const int slot = (G - o - 1 + KS) % KS;
                        int32_t *xo = xch + (((sub * KS + o) * (KS - 1) + slot) * VPW) * 64 + lane;
#pragma unroll
                        for (int v = 0; v < VPW; v++) xo[64 * v] = isum[VPW * o + v];
                    }
                    lds_barrier();
                    // own part
                    int32_t mine[VPW];
#pragma unroll
                    for (int v = 0; v < VPW; v++) mine[v] = isum[VPW * G + v];
#pragma unroll
                    for (int sl = 0; sl < KS - 1; sl++) {
                        const int32_t *xi = xch + (((sub * KS + G) * (KS - 1) + sl) * VPW) * 64 + lane;
#pragma unroll
                        for (int v = 0; v < VPW; v++) mine[v] += xi[64 * v];
                    }

                    const float wd = s.wd[tn + col];
                    if constexpr (TYPE == 14) {
#pragma unroll
                        for (int v = 0; v < VPW; v++) {
                            const float yd = s.yd[tm + tok_of(VPW * G + v, h)];
                            sum[v] = __fadd_rn(sum[v], __fmul_rn(__fmul_rn(wd, yd), (float)mine[v]));
                        }
                    } else {
                        // isum_mins = sum_j m_j * (bsums[2j] + bsums[2j+1]) as two small
                        // MFMAs: the bsum pairs enter as int8 digits (lo | hi), the mins
                        // sit against the lo half for one product and the hi half for
                        // the other, so mins = lo_product + 128 * hi_product exactly.
                        const long amv = *(const QK_LDS long *)&s.am[tm + col][8 * h];
                        const long mnv = *(const QK_LDS long *)&s.mn[tn + col][0];
                        const v16i dl = __builtin_amdgcn_mfma_i32_32x32x16_i8(amv, h == 0 ? mnv : 0L, zero, 0, 0, 0);
                        const v16i dh = __builtin_amdgcn_mfma_i32_32x32x16_i8(amv, h == 1 ? mnv : 0L, zero, 0, 0, 0);
                        const float wdm = s.wdm[tn + col];
#pragma unroll
                        for (int v = 0; v < VPW; v++) {
                            const int vv = VPW * G + v;
                            const int32_t mins = dl[vv] + dh[vv] * 128;
                            const float yd = s.yd[tm + tok_of(vv, h)];
                            const float d = __fmul_rn(yd, wd);
                            const float dmin = __fmul_rn(yd, wdm);
                            const float pm = __fmul_rn(dmin, (float)mins);
                            const float term = FUSED ? __builtin_fmaf(d, (float)mine[v], -pm)
                                                     : __fsub_rn(__fmul_rn(d, (float)mine[v]), pm);
                            sum[v] = __fadd_rn(sum[v], term);
                        }
                    }
                };
                if (g == 0) finish(std::integral_constant<int, 0>{});
                else if (g == 1) finish(std::integral_constant<int, 1>{});
                else if (g == 2) finish(std::integral_constant<int, 2>{});
                else finish(std::integral_constant<int, 3>{});
            } else {
                // The KS waves of a sub-tile exchange parts: wave g finishes
                // outputs v = VPW*g .. VPW*g + VPW-1 and hands the others to
                // their owners. Integer sums: exact in any order.
                if (ALIAS) lds_barrier();                            // every wave is done reading s.a
#pragma unroll
                for (int o = 0; o < KS; o++) {
                    if (o == g) continue;
                    const int slot = (g - o - 1 + KS) % KS;
                    int32_t *xo = xch + (((sub * KS + o) * (KS - 1) + slot) * VPW) * 64 + lane;
#pragma unroll
                    for (int v = 0; v < VPW; v++) xo[64 * v] = isum[VPW * o + v];
                }
                lds_barrier();
                // own part (g is wave-uniform; selects keep every index static)
                int32_t mine[VPW];
#pragma unroll
                for (int v = 0; v < VPW; v++) {
                    mine[v] = isum[v];
#pragma unroll
                    for (int q = 1; q < KS; q++) mine[v] = g == q ? isum[VPW * q + v] : mine[v];
                }
#pragma unroll
                for (int sl = 0; sl < KS - 1; sl++) {
                    const int32_t *xi = xch + (((sub * KS + g) * (KS - 1) + sl) * VPW) * 64 + lane;
#pragma unroll
                    for (int v = 0; v < VPW; v++) mine[v] += xi[64 * v];
                }

                const float wd = s.wd[tn + col];
                if constexpr (TYPE == 14) {
#pragma unroll
                    for (int v = 0; v < VPW; v++) {
                        const float yd = s.yd[tm + tok_of(VPW * g + v, h)];
                        sum[v] = __fadd_rn(sum[v], __fmul_rn(__fmul_rn(wd, yd), (float)mine[v]));
                    }
                } else {
                    // isum_mins = sum_j m_j * (bsums[2j] + bsums[2j+1]) as two small
                    // MFMAs: the bsum pairs enter as int8 digits (lo | hi), the mins
                    // sit against the lo half for one product and the hi half for
                    // the other, so mins = lo_product + 128 * hi_product exactly.
                    const long amv = *(const QK_LDS long *)&s.am[tm + col][8 * h];
                    const long mnv = *(const QK_LDS long *)&s.mn[tn + col][0];
                    const v16i dl = __builtin_amdgcn_mfma_i32_32x32x16_i8(amv, h == 0 ? mnv : 0L, zero, 0, 0, 0);
                    const v16i dh = __builtin_amdgcn_mfma_i32_32x32x16_i8(amv, h == 1 ? mnv : 0L, zero, 0, 0, 0);
                    const float wdm = s.wdm[tn + col];
#pragma unroll
                    for (int v = 0; v < VPW; v++) {
                        const int vv = VPW * g + v;
                        int32_t ml = dl[v], mh = dh[v];
#pragma unroll
                        for (int q = 1; q < KS; q++) {
                            ml = g == q ? dl[VPW * q + v] : ml;
                            mh = g == q ? dh[VPW * q + v] : mh;
                        }
                        const int32_t mins = ml + mh * 128;
                        const float yd = s.yd[tm + tok_of(vv, h)];
                        const float d = __fmul_rn(yd, wd);
                        const float dmin = __fmul_rn(yd, wdm);
                        const float pm = __fmul_rn(dmin, (float)mins);
                        const float term = FUSED ? __builtin_fmaf(d, (float)mine[v], -pm)
                                                 : __fsub_rn(__fmul_rn(d, (float)mine[v]), pm);
                        sum[v] = __fadd_rn(sum[v], term);
                    }
                }
            }
        }

        // non-temporal stores: the outputs are not read again by this
        // kernel, and every workgroup's stores leave at about the same time
        const int64_t row = r0 + tn + col;
        if (row < n) store_mfma32<FUSED, VPW>(y, n, row, t0, tm, mrows, VPW * g, h, sum);
    };
    if (role == 1) {
        typename WRawOf<TYPE>::T wr;
        body(wr, std::integral_constant<int, 1>{});
    } else if (role == 0) {
        ActRaw ar;
        body(ar, std::integral_constant<int, 0>{});
    } else {
        NoRaw nr;
        body(nr, std::integral_constant<int, 2>{});
    }
}

// ---- wide token tiles (Q5_K) -------------------------------------------------------
// (Written for Q4_K and Q5_K; Q4_K now takes k_gemm_r at these lengths.)
// For prompts long enough to give many token tiles: a 512-thread workgroup
// owns 128 tokens x 64 weight rows, and wave w computes the 32x32 sub-tile
// at tokens 32*(w/2), rows 32*(w%2) over the whole super-block, so no int32
// parts are exchanged and each weight tile is unpacked once per 128 tokens.
// Every thread stages a quarter of one activation row and an eighth of one
// weight row: one 16-byte run of nibbles with both of its sub-blocks' scale
// digits, and one of the row's eight mins. The arithmetic per output is the
// 64-token kernel's.
#define GW_BM 128                     // tokens per wide tile

template <int NP>
struct __attribute__((aligned(16))) GemmWLds {
    int8_t a[GW_BM][GM_LD];           // activation quants of the super-block
    int8_t b[NP][64][GM_LD];          // dequantised int8 weight planes
    int8_t am[GW_BM][16];             // bsum pairs as two int8 digits
    float yd[GW_BM];                  // Q8_K d per token
    uint8_t mn[64][8];                // 6-bit mins
    float wd[64];                     // fp16 d, widened
    float wdm[64];                    // fp16 dmin, widened
};

// Eighth e of a Q4_K / Q5_K weight row: qs run q = e%4 of half e/4 (chunk
// c = 2*(e/4) + q/2, positions 16*(q&1)..+16), the header, and for Q5_K the
// qh bytes of those positions. Rows past n (row == nullptr) stage zeros.
struct WRawE { uint4 hdr, p, qh; };

template <int TYPE>
__device__ __forceinline__ void load_we(WRawE &a, const uint8_t *row, int e, int i) {
    a.hdr = a.p = a.qh = make_uint4(0, 0, 0, 0);
    if (!row) return;
    const int q = e & 3, half = e >> 2;
    if constexpr (TYPE == 12) {
        const uint8_t *p = row + (int64_t)i * Q4K_BYTES;
        a.hdr = ld16(p);
        a.p = ld16(p + 16 + 64 * half + 16 * q);
    } else {
        const uint8_t *p = row + (int64_t)i * Q5K_BYTES;
        a.hdr = ld16(p);
        a.qh = ld16(p + 16 + 16 * (q & 1));
        a.p = ld16(p + 48 + 64 * half + 16 * q);
    }
}

template <int TYPE, typename GL>
__device__ __forceinline__ void store_we(GL &s, const WRawE &a, int r, int e) {
    const int q = e & 3, c = 2 * (e >> 2) + (q >> 1), l0 = 16 * (q & 1);
    if constexpr (TYPE == 12) store_piece4(s, r, c, l0, a.p, a.hdr);
    else store_piece5(s, r, c, l0, a.p, a.qh, a.hdr);
    int32_t sc, mm;
    scale_min(a.hdr.y, a.hdr.z, a.hdr.w, e, sc, mm);
    s.mn[r][e] = (uint8_t)mm;
    if (e == 0) s.wd[r] = h2f(a.hdr.x & 0xffffu);
    if (e == 1) s.wdm[r] = h2f(a.hdr.x >> 16);
}

template <int TYPE, bool FUSED>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(TYPE == 12 ? 4 : 2)))
void k_gemm_w(const uint8_t *__restrict__ w, int64_t n, int nb, const uint8_t *__restrict__ xq, int64_t m,
              float *__restrict__ y) {
    constexpr int NP = Planes<TYPE>::n;
    constexpr int BB = TYPE == 12 ? Q4K_BYTES : Q5K_BYTES;
    __shared__ GemmWLds<NP> s;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int col = lane & 31, h = lane >> 5;
    const int tm = 32 * (wave >> 1), tn = 32 * (wave & 1);
    const int64_t r0 = (int64_t)blockIdx.x * 64, t0 = (int64_t)blockIdx.y * GW_BM;
    const int at = tid >> 2, aq = tid & 3;                   // activation row, quarter
    const int wt = tid >> 3, we = tid & 7;                   // weight row, eighth
    // activation rows of this token tile: one buffer of at most 128 x 256 x
    // 292 bytes, so every offset is 32-bit; rows past m read zeros
    const int mrows = (m - t0 < GW_BM) ? (int)(m - t0) : GW_BM;
    const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t *>(xq + t0 * nb * Q8K_BYTES), 0, mrows * nb * Q8K_BYTES, 0x00020000);
    const int xoff = at * nb * Q8K_BYTES;
    const uint8_t *wrow = r0 + wt < n ? w + (r0 + wt) * nb * BB : nullptr;

    ActRaw ar;
    WRawE wr;
    load_act(ar, xr, xoff, aq, 0);
    load_we<TYPE>(wr, wrow, we, 0);
    const int8_t *arow = &s.a[tm + col][0];
    const v16i zero = {0};
    float sum[16];
#pragma unroll
    for (int v = 0; v < 16; v++) sum[v] = 0.0f;
    for (int i = 0; i < nb; i++) {
        lds_barrier();                                       // previous super-block's reads done
        store_act(s, ar, at, aq);
        store_we<TYPE>(s, wr, wt, we);
        if (i + 1 < nb) {                                    // next super-block in flight during compute
            load_act(ar, xr, xoff, aq, i + 1);
            load_we<TYPE>(wr, wrow, we, i + 1);
        }
        lds_barrier();
        // one accumulation chain per digit plane over the super-block
        v16i acc[NP];
#pragma unroll
        for (int pl = 0; pl < NP; pl++) acc[pl] = zero;
#pragma unroll
        for (int c = 0; c < 8; c++) {
            const v4i av = *(const QK_LDS v4i *)(arow + 32 * c + 16 * h);
#pragma unroll
            for (int pl = 0; pl < NP; pl++) {
                const v4i bv = *(const QK_LDS v4i *)(&s.b[pl][tn + col][32 * c + 16 * h]);
                acc[pl] = __builtin_amdgcn_mfma_i32_32x32x32_i8(av, bv, acc[pl], 0, 0, 0);
            }
        }
        int32_t is[16];
#pragma unroll
        for (int v = 0; v < 16; v++) {
            is[v] = acc[0][v] + 8 * acc[1][v];
            if constexpr (NP == 3) is[v] += 16 * acc[2][v];
        }
        // isum_mins as two small MFMAs (bsum pair digits lo | hi against the
        // mins: mins = lo_product + 128 * hi_product exactly)
        const long amv = *(const QK_LDS long *)&s.am[tm + col][8 * h];
        const long mnv = *(const QK_LDS long *)&s.mn[tn + col][0];
        const v16i dl = __builtin_amdgcn_mfma_i32_32x32x16_i8(amv, h == 0 ? mnv : 0L, zero, 0, 0, 0);
        const v16i dh = __builtin_amdgcn_mfma_i32_32x32x16_i8(amv, h == 1 ? mnv : 0L, zero, 0, 0, 0);
        const float wd = s.wd[tn + col], wdm = s.wdm[tn + col];
#pragma unroll
        for (int v = 0; v < 16; v++) {
            const int32_t mins = dl[v] + dh[v] * 128;
            const float yd = s.yd[tm + tok_of(v, h)];
            const float d = __fmul_rn(yd, wd);
            const float dmin = __fmul_rn(yd, wdm);
            const float pm = __fmul_rn(dmin, (float)mins);
            const float term =
                FUSED ? __builtin_fmaf(d, (float)is[v], -pm) : __fsub_rn(__fmul_rn(d, (float)is[v]), pm);
            sum[v] = __fadd_rn(sum[v], term);
        }
    }
    const int64_t row = r0 + tn + col;
    if (row < n) store_mfma32<FUSED, 16>(y, n, row, t0, tm, mrows, 0, h, sum);
}

// ---- weight rows in registers (Q4_K) -----------------------------------------------
// A 256-thread workgroup owns TT tokens x 128 weight rows; wave w owns rows
// 32w..32w+31 for all TT tokens. Only the activations go through LDS (one
// 16-byte store per 16 bytes, shared by the four waves); each wave loads
// its weight rows straight into registers, lane l taking row l % 32 and
// the 16-byte qs runs of k-half l / 32: the run at 16 + 32c + 16h holds,
// in its low nibbles, elements 16h.. of sub-block 2c and, in its high
// nibbles, the same positions of sub-block 2c + 1 -- exactly the B operand
// bytes of the two MFMAs over those sub-blocks. The scale digits are
// multiplied in with packed 16-bit multiplies, in registers, so no weight
// byte is written to LDS. The arithmetic per output is k_gemm_w's.
template <bool FUSED, int TT>
__global__ __launch_bounds__(256) void k_gemm_r(const uint8_t *__restrict__ w, int64_t n, int nb,
                                                const uint8_t *__restrict__ xq, int64_t m, float *__restrict__ y) {
    constexpr int NT = TT / 32;                        // MFMA token tiles
    __shared__ __attribute__((aligned(16))) int8_t sa[TT][GM_LD];   // activation quants of the super-block
    __shared__ __attribute__((aligned(16))) int8_t sam[TT][16];     // bsum pairs as two int8 digits
    __shared__ float syd[TT];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int col = lane & 31, h = lane >> 5;
    const int64_t r0 = (int64_t)blockIdx.x * 128, t0 = (int64_t)blockIdx.y * TT;
    // activations: thread t stages eighth e = t % 8 (32 bytes, bsum pair e)
    // of tokens t / 8 + 32 j
    const int at = tid >> 3, ae = tid & 7;
    const int mrows = (m - t0 < TT) ? (int)(m - t0) : TT;
    const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t *>(xq + t0 * nb * Q8K_BYTES), 0, mrows * nb * Q8K_BYTES, 0x00020000);
    struct A8 { uint4 q0, q1; uint32_t bp, d; } ar[NT];
    // token at's byte offset in the tile (below 2^24: nb <= 256)
    const int abase = (int)__umul24((uint32_t)at, (uint32_t)(nb * Q8K_BYTES));
    auto load_a = [&](int i) {
#pragma unroll
        for (int j = 0; j < NT; j++) {
            const int o = abase + (32 * j * nb + i) * Q8K_BYTES;
            ar[j].q0 = bl128(xr, o + 4 + 32 * ae);
            ar[j].q1 = bl128(xr, o + 20 + 32 * ae);
            ar[j].bp = bl32(xr, o + 260 + 4 * ae);
            ar[j].d = bl32(xr, o);
        }
    };
    auto store_a = [&]() {
#pragma unroll
        for (int j = 0; j < NT; j++) {
            const int t = at + 32 * j;
            *(QK_LDS uint4 *)&sa[t][32 * ae] = ar[j].q0;
            *(QK_LDS uint4 *)&sa[t][32 * ae + 16] = ar[j].q1;
            const int32_t p = (int32_t)(int16_t)(ar[j].bp & 0xffffu) + (int32_t)(int16_t)(ar[j].bp >> 16);
            sam[t][ae] = (int8_t)(p & 127);
            sam[t][8 + ae] = (int8_t)(p >> 7);
            if (ae == 0) syd[t] = __uint_as_float(ar[j].d);
        }
    };
    // weights: this lane's row and k-half
    const int64_t row = r0 + 32 * wave + col;
    const uint8_t *wp = row < n ? w + (uint64_t)(uint32_t)row * (uint32_t)(nb * Q4K_BYTES) : nullptr;
    struct W5 { uint4 hdr, p[4]; } wr;
    auto load_w = [&](int i) {
        if (!wp) {
            wr.hdr = make_uint4(0, 0, 0, 0);
#pragma unroll
            for (int c = 0; c < 4; c++) wr.p[c] = make_uint4(0, 0, 0, 0);
            return;
        }
        const uint8_t *p = wp + (int64_t)i * Q4K_BYTES;
        wr.hdr = ld16(p);
#pragma unroll
        for (int c = 0; c < 4; c++) wr.p[c] = ld16(p + 16 + 32 * c + 16 * h);
    };
    load_a(0);
    load_w(0);
    const v16i zero = {0};
    float sum[NT][16];
#pragma unroll
    for (int j = 0; j < NT; j++)
#pragma unroll
        for (int v = 0; v < 16; v++) sum[j][v] = 0.0f;
    for (int i = 0; i < nb; i++) {
        lds_barrier();                                 // previous super-block's reads done
        store_a();
        const W5 cw = wr;                              // this super-block's weight bytes
        if (i + 1 < nb) {                              // the next one in flight during compute
            load_a(i + 1);
            load_w(i + 1);
        }
        lds_barrier();
        // this super-block's B operands: the two digit planes of every
        // sub-block, and the mins operand
        v4i pb[8][2];
        uint32_t mn[8];                                // 6-bit mins
#pragma unroll
        for (int c = 0; c < 4; c++) {
            const uint32_t M = 0x0F0F0F0Fu;
            const uint4 v = cw.p[c];
            const uint32_t q[2][4] = {{v.x & M, v.y & M, v.z & M, v.w & M},
                                      {(v.x >> 4) & M, (v.y >> 4) & M, (v.z >> 4) & M, (v.w >> 4) & M}};
#pragma unroll
            for (int hs = 0; hs < 2; hs++) {           // sub-block 2c + hs
                const int sb = 2 * c + hs;
                int32_t sc, mm;
                scale_min(cw.hdr.y, cw.hdr.z, cw.hdr.w, sb, sc, mm);
                mn[sb] = (uint32_t)mm;
                const uint32_t lo = (uint32_t)sc & 7u, hi = (uint32_t)sc >> 3;
                pb[sb][0] = v4i{(int)bmul(q[hs][0], lo), (int)bmul(q[hs][1], lo), (int)bmul(q[hs][2], lo),
                                (int)bmul(q[hs][3], lo)};
                pb[sb][1] = v4i{(int)bmul(q[hs][0], hi), (int)bmul(q[hs][1], hi), (int)bmul(q[hs][2], hi),
                                (int)bmul(q[hs][3], hi)};
            }
        }
        const long mnv = (long)((uint64_t)mn[0] | (uint64_t)mn[1] << 8 | (uint64_t)mn[2] << 16 |
                                (uint64_t)mn[3] << 24 | (uint64_t)mn[4] << 32 | (uint64_t)mn[5] << 40 |
                                (uint64_t)mn[6] << 48 | (uint64_t)mn[7] << 56);
        const float wd = h2f(cw.hdr.x & 0xffffu), wdm = h2f(cw.hdr.x >> 16);
        // token tile j's products, then its fp32 terms; the products of
        // tile j + 1 come first in the order, beside tile j's terms
        v16i a0[NT], a1[NT], dl[NT], dh[NT];
        auto products = [&](int j) {
            a0[j] = a1[j] = zero;
#pragma unroll
            for (int sb = 0; sb < 8; sb++) {
                const v4i av = *(const QK_LDS v4i *)(&sa[32 * j + col][32 * sb + 16 * h]);
                a0[j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(av, pb[sb][0], a0[j], 0, 0, 0);
                a1[j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(av, pb[sb][1], a1[j], 0, 0, 0);
            }
            // isum_mins as two small MFMAs (bsum pair digits lo | hi
            // against the mins: mins = lo_product + 128 * hi_product)
            const long amv = *(const QK_LDS long *)&sam[32 * j + col][8 * h];
            dl[j] = __builtin_amdgcn_mfma_i32_32x32x16_i8(amv, h == 0 ? mnv : 0L, zero, 0, 0, 0);
            dh[j] = __builtin_amdgcn_mfma_i32_32x32x16_i8(amv, h == 1 ? mnv : 0L, zero, 0, 0, 0);
        };
        auto terms = [&](int j) {
#pragma unroll
            for (int v = 0; v < 16; v++) {
                const int32_t is = a0[j][v] + 8 * a1[j][v];
                const int32_t mins = dl[j][v] + dh[j][v] * 128;
                const float yd = syd[32 * j + tok_of(v, h)];
                const float d = __fmul_rn(yd, wd);
                const float dmin = __fmul_rn(yd, wdm);
                const float pm = __fmul_rn(dmin, (float)mins);
                const float term =
                    FUSED ? __builtin_fmaf(d, (float)is, -pm) : __fsub_rn(__fmul_rn(d, (float)is), pm);
                sum[j][v] = __fadd_rn(sum[j][v], term);
            }
        };
        products(0);
#pragma unroll
        for (int j = 1; j < NT; j++) {
            products(j);
            terms(j - 1);
        }
        terms(NT - 1);
    }
    if (row < n) {
#pragma unroll
        for (int j = 0; j < NT; j++) store_mfma32<FUSED, 16>(y, n, row, t0, 32 * j, mrows, 0, h, sum[j]);
    }
}

// ---- super-blocks across waves (Q4_K, short prompts) ---------------------------
// A 256-thread workgroup owns one 32-token x 32-row output tile; in round
// r its wave w computes super-block 4r + w, so the waves of a workgroup run
// the super-blocks of a tile side by side instead of one after another.
// The super-block terms are formed exactly as in k_gemm_r (lane l: row
// l % 32, k-half l / 32) and then summed in super-block order: every wave
// writes its 16 terms per lane to LDS, and wave w adds, for outputs
// 4w..4w+3 of every lane, the round's terms in order to the running sums
// (sum starts at +0.0, so the first term enters exactly), which is the
// reference's sequential `sum += term`. SHARE: the terms reuse the
// activations' LDS once every wave has read them (one more barrier a
// round), so four workgroups fit a CU instead of three.
template <bool SHARE> struct KsShared {
    int8_t sa[4][32][GM_LD];          // super-block 4r + q in sa[q]: a token's 256 quants, then its bsum pairs as two int8 digits
    float st[4][16][64];              // st[q][v][lane]: wave q's term for output v of a lane
};
template <> struct KsShared<true> {
    union { int8_t sa[4][32][GM_LD]; float st[4][16][64]; };
};

template <bool FUSED, bool SHARE>
__global__ __launch_bounds__(256) void k_gemm_ks(const uint8_t *__restrict__ w, int64_t n, int nb,
                                                 const uint8_t *__restrict__ xq, int64_t m, float *__restrict__ y) {
    __shared__ __attribute__((aligned(16))) KsShared<SHARE> sh;
    __shared__ float syd[4][32];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int col = lane & 31, h = lane >> 5;
    const int64_t r0 = (int64_t)blockIdx.x * 32, t0 = (int64_t)blockIdx.y * 32;
    const int mrows = (m - t0 < 32) ? (int)(m - t0) : 32;
    const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t *>(xq + t0 * nb * Q8K_BYTES), 0, mrows * nb * Q8K_BYTES, 0x00020000);
    // staging: thread t stages eighth e = t % 8 of token t / 8 for each of
    // the round's four super-blocks; the token's byte offset in the tile
    // (below 2^24: nb <= 256)
    const int at = tid >> 3, ae = tid & 7;
    const int abase = (int)__umul24((uint32_t)at, (uint32_t)(nb * Q8K_BYTES)) + 32 * ae;
    const int64_t row = r0 + col;
    const uint32_t rowc = (uint32_t)(row < n ? row : n - 1);
    const uint8_t *wp = w + (uint64_t)rowc * (uint32_t)(nb * Q4K_BYTES) + 16 * h;
    const v16i zero = {0};
    float sum[4] = {0.0f, 0.0f, 0.0f, 0.0f};          // this lane's outputs v = 4 * wave + b
    for (int r = 0; r < nb; r += 4) {
        const int sb = r + wave;                       // this wave's super-block
        const bool act = sb < nb;                      // wave-uniform
        // weights of this wave's super-block, in flight during staging
        struct W5 { uint4 hdr, p[4]; } cw;
        {
            const uint8_t *p = wp + (act ? sb : nb - 1) * Q4K_BYTES;
            cw.hdr = ld16(p - 16 * h);
#pragma unroll
            for (int c = 0; c < 4; c++) cw.p[c] = ld16(p + 16 + 32 * c);
        }
        // the round's activations, in flight during the unpack
        struct A8 { uint4 q0, q1; uint32_t bp, d; } ar[4];
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const int o = abase + (r + q < nb ? r + q : nb - 1) * Q8K_BYTES;
            ar[q].q0 = bl128(xr, o + 4);
            ar[q].q1 = bl128(xr, o + 20);
            ar[q].bp = bl32(xr, o + 260 - 28 * ae);
            ar[q].d = bl32(xr, o - 32 * ae);
        }
        // previous round's reads done, then this round's activations
        auto stage = [&]() {
            if (r > 0) lds_barrier();
#pragma unroll
            for (int q = 0; q < 4; q++) {
                if (r + q >= nb) break;                // uniform
                *(QK_LDS uint4 *)&sh.sa[q][at][32 * ae] = ar[q].q0;
                *(QK_LDS uint4 *)&sh.sa[q][at][32 * ae + 16] = ar[q].q1;
                const int32_t pr = (int32_t)(int16_t)(ar[q].bp & 0xffffu) + (int32_t)(int16_t)(ar[q].bp >> 16);
                sh.sa[q][at][256 + ae] = (int8_t)(pr & 127);
                sh.sa[q][at][264 + ae] = (int8_t)(pr >> 7);
                if (ae == 0) syd[q][at] = __uint_as_float(ar[q].d);
            }
            lds_barrier();
        };
        float tm[16];                                  // this wave's terms
        if (!act) stage();                             // wave-uniform: the barriers match the active waves'
        if (act) {
            v4i pb[8][2];
            uint32_t mn[8];
#pragma unroll
            for (int c = 0; c < 4; c++) {
                const uint32_t M = 0x0F0F0F0Fu;
                const uint4 v = cw.p[c];
                const uint32_t q[2][4] = {{v.x & M, v.y & M, v.z & M, v.w & M},
                                          {(v.x >> 4) & M, (v.y >> 4) & M, (v.z >> 4) & M, (v.w >> 4) & M}};
#pragma unroll
                for (int hs = 0; hs < 2; hs++) {
                    const int s2 = 2 * c + hs;
                    int32_t sc, mm;
                    scale_min(cw.hdr.y, cw.hdr.z, cw.hdr.w, s2, sc, mm);
                    mn[s2] = (uint32_t)mm;
                    const uint32_t lo = (uint32_t)sc & 7u, hi = (uint32_t)sc >> 3;
                    pb[s2][0] = v4i{(int)bmul(q[hs][0], lo), (int)bmul(q[hs][1], lo), (int)bmul(q[hs][2], lo),
                                    (int)bmul(q[hs][3], lo)};
                    pb[s2][1] = v4i{(int)bmul(q[hs][0], hi), (int)bmul(q[hs][1], hi), (int)bmul(q[hs][2], hi),
                                    (int)bmul(q[hs][3], hi)};
                }
            }
            const long mnv = (long)((uint64_t)mn[0] | (uint64_t)mn[1] << 8 | (uint64_t)mn[2] << 16 |
                                    (uint64_t)mn[3] << 24 | (uint64_t)mn[4] << 32 | (uint64_t)mn[5] << 40 |
                                    (uint64_t)mn[6] << 48 | (uint64_t)mn[7] << 56);
            const float wd = h2f(cw.hdr.x & 0xffffu), wdm = h2f(cw.hdr.x >> 16);
            stage();
            v16i a0 = zero, a1 = zero;
#pragma unroll
            for (int s2 = 0; s2 < 8; s2++) {
                const v4i av = *(const QK_LDS v4i *)(&sh.sa[wave][col][32 * s2 + 16 * h]);
                a0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(av, pb[s2][0], a0, 0, 0, 0);
                a1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(av, pb[s2][1], a1, 0, 0, 0);
            }
            // isum_mins as two small MFMAs (bsum pair digits lo | hi
            // against the mins: mins = lo_product + 128 * hi_product)
            const long amv = *(const QK_LDS long *)&sh.sa[wave][col][256 + 8 * h];
            const v16i dl = __builtin_amdgcn_mfma_i32_32x32x16_i8(amv, h == 0 ? mnv : 0L, zero, 0, 0, 0);
            const v16i dh = __builtin_amdgcn_mfma_i32_32x32x16_i8(amv, h == 1 ? mnv : 0L, zero, 0, 0, 0);
#pragma unroll
            for (int v = 0; v < 16; v++) {
                const int32_t is = a0[v] + 8 * a1[v];
                const int32_t mins = dl[v] + dh[v] * 128;
                const float yd = syd[wave][tok_of(v, h)];
                const float d = __fmul_rn(yd, wd);
                const float dmin = __fmul_rn(yd, wdm);
                const float pm = __fmul_rn(dmin, (float)mins);
                tm[v] = FUSED ? __builtin_fmaf(d, (float)is, -pm) : __fsub_rn(__fmul_rn(d, (float)is), pm);
            }
        }
        if constexpr (SHARE) lds_barrier();            // every wave's reads of sa done
        if (act) {
#pragma unroll
            for (int v = 0; v < 16; v++) sh.st[wave][v][lane] = tm[v];
        }
        lds_barrier();
        // the round's terms in super-block order, outputs 4 * wave .. + 3
#pragma unroll
        for (int q = 0; q < 4; q++) {
            if (r + q >= nb) break;                    // uniform
#pragma unroll
            for (int b = 0; b < 4; b++) sum[b] = __fadd_rn(sum[b], sh.st[q][4 * wave + b][lane]);
        }
    }
    if (row < n) store_mfma32<FUSED, 4>(y, n, row, t0, 0, mrows, 4 * wave, h, sum);
}
// ---- super-blocks across waves (Q6_K) -------------------------------------------
// k_gemm_ks for Q6_K (q6k_row_dot_q8k, simd/quants.h:355-402): a 256-thread
// workgroup owns one 32-token x 32-row tile, wave w computes super-block
// 4r + w in round r, and the waves' fp32 terms are added in super-block
// order through LDS. Per super-block, the reference's integer sums:
//
//  * isum = sum_j scale_j * sum_{e in sub-block j} w_e * y_e over the
//    unsigned 6-bit weights w: one v_mfma_i32_32x32x16_i8 per 16-element
//    sub-block (lane half h takes elements 8h..8h+7 of it, in both
//    operands), times the row's int8 scale, added in int32 (exact);
//  * isum_mins = sum_j bsums_j * scale_j: one v_mfma_f32_32x32x16_f16,
//    every operand exact in f16 (|bsums_j| <= 16 * 128 = 2048, the
//    magnitude any Q8_K block's sixteen quants give) and every partial sum
//    an integer below 2^24, so exact in f32;
//
// then term = rn(rn(fp16(d) * y.d) * (float)(isum - 32 * isum_mins)).
// Element 16jj + l (l < 16) of a 128-element half hb is the low (jj < 4)
// or high nibble of ql[64hb + 16(jj % 4) + l] with bits 2(jj / 2).. of
// qh[32hb + 16(jj % 2) + l] on top, so lane half h reads 8-byte runs at
// 64hb + 16c + 8h (c < 4) and 128 + 32hb + 16c + 8h (c < 2): twelve runs,
// each through the three aligned dwords that contain it (blocks are
// 2-byte aligned).
// S waves per workgroup, S super-blocks per round (4 or 8). With 8, the
// waves' terms reuse the activations' LDS once every wave has read them
// (one more barrier), so two workgroups fit a CU.
template <int S> struct Ks6Tiles { int8_t sa[S][32][GM_LD]; float st[S][16][64]; };
template <int S> union Ks6Shared { int8_t sa[S][32][GM_LD]; float st[S][16][64]; };

template <bool FUSED, int S>
__global__ __launch_bounds__(64 * S) void k_gemm_ks6(const uint8_t *__restrict__ w, int64_t n, int nb,
                                                  const uint8_t *__restrict__ xq, int64_t m, float *__restrict__ y) {
    // super-block Sr + q in sa[q]; the waves' terms in st[wave][v][lane]
    constexpr bool ALIAS = S == 8;
    __shared__ __attribute__((aligned(16))) std::conditional_t<ALIAS, Ks6Shared<S>, Ks6Tiles<S>> u;
    auto &sa = u.sa;
    auto &st = u.st;
    __shared__ __attribute__((aligned(16))) _Float16 sbs[S][32][16];   // its bsums in f16
    __shared__ float syd[S][32];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int col = lane & 31, h = lane >> 5;
    const int64_t r0 = (int64_t)blockIdx.x * 32, t0 = (int64_t)blockIdx.y * 32;
    const int mrows = (m - t0 < 32) ? (int)(m - t0) : 32;
    const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t *>(xq + t0 * nb * Q8K_BYTES), 0, mrows * nb * Q8K_BYTES, 0x00020000);
    // the tile's weight rows as one buffer from the 4-byte aligned address
    // at or below its first row; rows past n read zeros
    const int nrows = (n - r0 < 32) ? (int)(n - r0) : 32;
    const uint8_t *wt = w + r0 * nb * Q6K_BYTES;
    const int off0 = (int)(reinterpret_cast<uintptr_t>(wt) & 3u);
    const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t *>(wt - off0), 0, off0 + nrows * nb * Q6K_BYTES, 0x00020000);
    // staging: eighth ae of token at, of super-blocks Sr + 4g .. + 3
    const int at = (tid >> 3) & 31, ae = tid & 7, ag = tid >> 8;
    const int abase = (int)__umul24((uint32_t)at, (uint32_t)(nb * Q8K_BYTES));   // below 2^24: nb <= 256
    const int row = (int)(r0 + col);
    constexpr int VW = 16 / S;                         // outputs per lane each wave adds up
    float sum[VW];
#pragma unroll
    for (int bb = 0; bb < VW; bb++) sum[bb] = 0.0f;
    const v16i zero = {0};
    for (int r = 0; r < nb; r += S) {
        const int sb = r + wave;
        const bool act = sb < nb;                      // wave-uniform
        // this wave's super-block: twelve 8-byte runs, the scales and d
        const int b = off0 + (col * nb + (act ? sb : nb - 1)) * Q6K_BYTES;
        const int sh = b & 3, ba = b - sh;
        uint32_t raw[12][3], rs[5], rd;
#pragma unroll
        for (int hb = 0; hb < 2; hb++) {
#pragma unroll
            for (int c = 0; c < 4; c++) {
                const auto v = __builtin_amdgcn_raw_buffer_load_b96(wr, ba + 64 * hb + 16 * c + 8 * h, 0, 0);
                raw[6 * hb + c][0] = v[0], raw[6 * hb + c][1] = v[1], raw[6 * hb + c][2] = v[2];
            }
#pragma unroll
            for (int c = 0; c < 2; c++) {
                const auto v = __builtin_amdgcn_raw_buffer_load_b96(wr, ba + 128 + 32 * hb + 16 * c + 8 * h, 0, 0);
                raw[6 * hb + 4 + c][0] = v[0], raw[6 * hb + 4 + c][1] = v[1], raw[6 * hb + 4 + c][2] = v[2];
            }
        }
        {
            const uint4 v = bl128(wr, ba + 192);
            rs[0] = v.x, rs[1] = v.y, rs[2] = v.z, rs[3] = v.w;
            rs[4] = bl32(wr, ba + 208);                // used only when sh > 0, then inside the block
            rd = __builtin_amdgcn_raw_buffer_load_b16(wr, b + 208, 0, 0);
        }
        // the round's activations, in flight during the unpack
        struct A8 { uint4 q0, q1; uint32_t bp, d; } ar[4];
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const int sq = r + 4 * ag + q;
            const int o = abase + (sq < nb ? sq : nb - 1) * Q8K_BYTES;
            ar[q].q0 = bl128(xr, o + 4 + 32 * ae);
            ar[q].q1 = bl128(xr, o + 20 + 32 * ae);
            ar[q].bp = bl32(xr, o + 260 + 4 * ae);
            ar[q].d = bl32(xr, o);
        }
        auto stage = [&]() {
            if (r > 0) lds_barrier();                  // the previous round's reads of st done
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const int qq = 4 * ag + q;
                if (r + qq >= nb) break;               // wave-uniform
                *(QK_LDS uint4 *)&sa[qq][at][32 * ae] = ar[q].q0;
                *(QK_LDS uint4 *)&sa[qq][at][32 * ae + 16] = ar[q].q1;
                sbs[qq][at][2 * ae] = (_Float16)(int16_t)(ar[q].bp & 0xffffu);
                sbs[qq][at][2 * ae + 1] = (_Float16)(int16_t)(ar[q].bp >> 16);
                if (ae == 0) syd[qq][at] = __uint_as_float(ar[q].d);
            }
            lds_barrier();
        };
        if (!act) {                                    // wave-uniform: the barriers match the active waves'
            stage();
            if constexpr (ALIAS) lds_barrier();
        }
        if (act) {
            // runs realigned, then the sixteen B operands (unsigned 6-bit)
            uint32_t run[12][2];
#pragma unroll
            for (int k = 0; k < 12; k++) {
                run[k][0] = __builtin_amdgcn_alignbyte(raw[k][1], raw[k][0], sh);
                run[k][1] = __builtin_amdgcn_alignbyte(raw[k][2], raw[k][1], sh);
            }
            long bq[16];
#pragma unroll
            for (int hb = 0; hb < 2; hb++)
#pragma unroll
                for (int jj = 0; jj < 8; jj++) {
                    uint32_t qd[2];
#pragma unroll
                    for (int k = 0; k < 2; k++) {
                        const uint32_t lo = (run[6 * hb + (jj & 3)][k] >> (4 * (jj >> 2))) & 0x0F0F0F0Fu;
                        const uint32_t hi = ((run[6 * hb + 4 + (jj & 1)][k] >> (2 * (jj >> 1))) & 0x03030303u) << 4;
                        qd[k] = lo | hi;
                    }
                    bq[8 * hb + jj] = (long)((uint64_t)qd[0] | ((uint64_t)qd[1] << 32));
                }
            uint32_t scw[4];
#pragma unroll
            for (int k = 0; k < 4; k++) scw[k] = __builtin_amdgcn_alignbyte(rs[k + 1], rs[k], sh);
            const float wd = h2f(rd);
            // mins operand: scales 8h..8h+7 in f16
            v8h mb;
#pragma unroll
            for (int k = 0; k < 8; k++) mb[k] = (_Float16)(int8_t)(scw[2 * h + (k >> 2)] >> (8 * (k & 3)));
            stage();
            int32_t isum[16];
#pragma unroll
            for (int v = 0; v < 16; v++) isum[v] = 0;
#pragma unroll
            for (int j = 0; j < 16; j++) {
                const long av = *(const QK_LDS long *)&sa[wave][col][16 * j + 8 * h];
                const v16i d = __builtin_amdgcn_mfma_i32_32x32x16_i8(av, bq[j], zero, 0, 0, 0);
                const int32_t scv = (int32_t)(int8_t)(scw[j >> 2] >> (8 * (j & 3)));
#pragma unroll
                for (int v = 0; v < 16; v++) isum[v] += __mul24(scv, d[v]);
            }
            const v8h amv = *(const QK_LDS v8h *)&sbs[wave][col][8 * h];
            const v16f mf = __builtin_amdgcn_mfma_f32_32x32x16_f16(amv, mb, v16f{0.0f}, 0, 0, 0);
            if constexpr (ALIAS) lds_barrier();        // every wave's reads of sa done: st reuses it
#pragma unroll
            for (int v = 0; v < 16; v++) {
                const int32_t is = isum[v] - 32 * (int32_t)mf[v];
                const float yd = syd[wave][tok_of(v, h)];
                st[wave][v][lane] = __fmul_rn(__fmul_rn(wd, yd), (float)is);
            }
        }
        lds_barrier();
        // the round's terms in super-block order, outputs VW * wave ..
#pragma unroll
        for (int q = 0; q < S; q++) {
            if (r + q >= nb) break;                    // uniform
#pragma unroll
            for (int bb = 0; bb < VW; bb++) sum[bb] = __fadd_rn(sum[bb], st[q][VW * wave + bb][lane]);
        }
    }
    if (row < n) store_mfma32<FUSED, VW>(y, n, row, t0, 0, mrows, VW * wave, h, sum);
}

// ---- Q8_0 x Q8_0 --------------------------------------------------------------
// The token loop of tensor_matmul_q8_0_f32 (slm/tensor.c:952-981) over
// q8_0_dot_q8_0 (simd/avx.c:65-158, simd/quants.h:244-256). Per 32-element
// block the AVX2/VNNI tiers keep eight int32 slot partials p_s (bytes
// 4s..4s+3) and eight fp32 chains acc_s = fma((float)p_s, d_w*d_x, acc_s),
// summed at the end as ((a0+a4)+(a1+a5)) + ((a2+a6)+(a3+a7)); the scalar
// and AVX1 tiers add (float)(sum of the block) * (d_w*d_x) to one sum.
//
// One v_mfma_i32_32x32x32_i8 covers one block (K = 32) of 4 weight rows x
// 32 tokens with every slot apart: its 32 A rows are (weight row j, slot
// s) = 8j + s, each the weight row's block with every byte outside slot s
// zeroed. Output v of a lane is then p_s of row j = v/4, slot
// s = 4h + v%4 (h = lane/32) for token lane%32, so the lane runs the fp32
// chains of four slots of four rows; the other four slots sit in lane
// l^32. The mask selects bytes by their position in the staged block,
// and both operands of a lane hold the same block positions, so it does
// not depend on the MFMA's internal k order.
//
// A 512-thread workgroup owns RT weight rows x TT tokens (32 x 32) and
// walks the blocks in steps of 8: the step's blocks are staged into LDS
// (quants at a 16-byte aligned stride, d widened) while the next step's
// raw bytes load into registers. Its RT/4 x TT/32 MFMA tiles per block are spread
// over the eight waves; each tile is one chain of MFMA, conversion and
// FMAs per block, so the tiles of several waves per SIMD overlap.
#define G8_KB 8                       // blocks per step
#define G8_LD (G8_KB * 32 + 16)       // LDS row stride of the quants

template <int RT, int TT>
struct __attribute__((aligned(16))) Gemm80Lds {
    int8_t w[RT][G8_LD];              // weight quants of the step's blocks
    int8_t x[TT][G8_LD];              // activation quants
    float wd[G8_KB][RT];              // weight d, rows contiguous
    float xd[G8_KB][TT];              // activation d
};

// One 34-byte block (d | qs[32]) at byte offset o of a buffer whose base
// is 4-byte aligned: qs through the nine aligned dwords that contain it
// (o is even, so the shift is 0 or 2), d as a 16-bit load.
struct Q80Raw { uint4 a, b; uint32_t c, d, sh; };

__device__ __forceinline__ void load_q80(Q80Raw &r, __amdgpu_buffer_rsrc_t rs, int o) {
    const int q = o + 2, a = q & ~3;
    r.sh = (uint32_t)(q & 3);
    r.a = bl128(rs, a);
    r.b = bl128(rs, a + 16);
    r.c = bl32(rs, a + 32);
    r.d = __builtin_amdgcn_raw_buffer_load_b16(rs, o, 0, 0);
}

__device__ __forceinline__ void store_q80(const Q80Raw &r, int8_t *qs, float *d) {
    const uint32_t v[9] = {r.a.x, r.a.y, r.a.z, r.a.w, r.b.x, r.b.y, r.b.z, r.b.w, r.c};
    uint32_t q[8];
#pragma unroll
    for (int i = 0; i < 8; i++) q[i] = __builtin_amdgcn_alignbyte(v[i + 1], v[i], r.sh);
    lds_st16(qs, q[0], q[1], q[2], q[3]);
    lds_st16(qs + 16, q[4], q[5], q[6], q[7]);
    *d = h2f(r.d);
}

template <bool FUSED, int RT, int TT>
__global__ __launch_bounds__(512) void k_gemm_q80(const uint8_t *__restrict__ w, int64_t n, int nb,
                                                  const uint8_t *__restrict__ xq, int64_t m,
                                                  float *__restrict__ y) {
    constexpr int NRG = RT / 4, NTH = TT / 32;           // 4-row groups, 32-token halves
    constexpr int TPW = NRG * NTH / 8;                   // MFMA tiles per wave
    constexpr int NPAIR = (RT + TT) * G8_KB;             // (row or token, block) pairs per step
    constexpr int NSLOT = (NPAIR + 511) / 512;           // of them per thread
    static_assert(TPW >= 1 && NRG * NTH == 8 * TPW, "tiles split evenly over 8 waves");
    static_assert((RT * G8_KB) % 64 == 0, "a wave stages weights or activations, not both");
    __shared__ Gemm80Lds<RT, TT> s;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int col = lane & 31, h = lane >> 5;
    const int64_t r0 = (int64_t)blockIdx.x * RT, t0 = (int64_t)blockIdx.y * TT;
    const int rowb = nb * Q80_BYTES;
    // the tile's weight rows and tokens as buffers based at the 4-byte
    // aligned address at or below their first byte, ending at the 4-byte
    // boundary at or after their last byte (the same dwords hold both
    // ends), so rows past n and tokens past m read zeros
    const int nrows = (n - r0 < RT) ? (int)(n - r0) : RT;
    const int mrows = (m - t0 < TT) ? (int)(m - t0) : TT;
    const uint8_t *wt = w + r0 * rowb, *xt = xq + t0 * rowb;
    const int wmis = (int)(reinterpret_cast<uintptr_t>(wt) & 3u), xmis = (int)(reinterpret_cast<uintptr_t>(xt) & 3u);
    const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t *>(wt - wmis), 0, (wmis + nrows * rowb + 3) & ~3, 0x00020000);
    const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t *>(xt - xmis), 0, (xmis + mrows * rowb + 3) & ~3, 0x00020000);
    // staging: pair p = tid + 512u is weight row p/8 (p < 8 RT) or token
    // p/8 - RT, block p%8 of the step (wave-uniform: 8 RT is a multiple of 64)
    Q80Raw raw[NSLOT];
    int so[NSLOT];
    auto load_step = [&](int b0) __attribute__((always_inline)) {
#pragma unroll
        for (int u = 0; u < NSLOT; u++) {
            const int p = tid + 512 * u;
            if (p < NPAIR) load_q80(raw[u], p < RT * G8_KB ? wr : xr, so[u] + b0 * Q80_BYTES);
        }
    };
#pragma unroll
    for (int u = 0; u < NSLOT; u++) {
        const int p = tid + 512 * u, r = p >> 3, kb = p & 7;
        so[u] = p < RT * G8_KB ? wmis + r * rowb + kb * Q80_BYTES : xmis + (r - RT) * rowb + kb * Q80_BYTES;
    }
    load_step(0);
    // this lane's slot (A row 8j + s, s = col % 8) as a mask of the four
    // dwords it holds (block bytes 16h..16h+15)
    const int sl = (col & 7) - 4 * h;
    const uint32_t mk0 = sl == 0 ? ~0u : 0u, mk1 = sl == 1 ? ~0u : 0u;
    const uint32_t mk2 = sl == 2 ? ~0u : 0u, mk3 = sl == 3 ? ~0u : 0u;
    const v16i zero = {0};
    // the wave's tiles: q = TPW * wave + i, row group q % NRG, token half q / NRG
    float acc[TPW][16];
#pragma unroll
    for (int i = 0; i < TPW; i++)
#pragma unroll
        for (int v = 0; v < 16; v++) acc[i][v] = 0.0f;

    for (int b0 = 0; b0 < nb; b0 += G8_KB) {
        lds_barrier();                                   // previous step's reads done
#pragma unroll
        for (int u = 0; u < NSLOT; u++) {
            const int p = tid + 512 * u, r = p >> 3, kb = p & 7;
            if (p < RT * G8_KB) store_q80(raw[u], &s.w[r][32 * kb], &s.wd[kb][r]);
            else if (p < NPAIR) store_q80(raw[u], &s.x[r - RT][32 * kb], &s.xd[kb][r - RT]);
        }
        if (b0 + G8_KB < nb) load_step(b0 + G8_KB);      // next step in flight during compute
        lds_barrier();
        const int kn = (nb - b0 < G8_KB) ? nb - b0 : G8_KB;
        // unrolled with a uniform guard: every LDS address is an immediate
        // offset from one base
#pragma unroll
        for (int kb = 0; kb < G8_KB; kb++) {
            if (kb >= kn) break;
#pragma unroll
            for (int i = 0; i < TPW; i++) {
                const int q = TPW * wave + i, rg = q % NRG, th = q / NRG;
                const v4i bx = *(const QK_LDS v4i *)&s.x[32 * th + col][32 * kb + 16 * h];
                const float dx = s.xd[kb][32 * th + col];
                const v4i aw = *(const QK_LDS v4i *)&s.w[4 * rg + (col >> 3)][32 * kb + 16 * h];
                const v4i am = {(int32_t)((uint32_t)aw[0] & mk0), (int32_t)((uint32_t)aw[1] & mk1),
                                (int32_t)((uint32_t)aw[2] & mk2), (int32_t)((uint32_t)aw[3] & mk3)};
                const float4 dw = *(const QK_LDS float4 *)&s.wd[kb][4 * rg];
                const float dwj[4] = {dw.x, dw.y, dw.z, dw.w};
                const v16i pr = __builtin_amdgcn_mfma_i32_32x32x32_i8(FUSED ? am : aw, bx, zero, 0, 0, 0);
                float *a = acc[i];
                if constexpr (FUSED) {
#pragma unroll
                    for (int j = 0; j < 4; j++) {
                        const float sc = __fmul_rn(dwj[j], dx);
#pragma unroll
                        for (int c = 0; c < 4; c++) a[4 * j + c] = __builtin_fmaf((float)pr[4 * j + c], sc, a[4 * j + c]);
                    }
                } else {
                    // unmasked A: every A row 8j + s is the whole block of row
                    // j, so its output is the block's sum (the same for all
                    // eight s); a[j] keeps row j's sum
#pragma unroll
                    for (int j = 0; j < 4; j++) {
                        const float sc = __fmul_rn(dwj[j], dx);
                        a[j] = __fadd_rn(a[j], __fmul_rn((float)pr[4 * j], sc));
                    }
                }
            }
        }
    }

    // lane h = 0 of token col stores rows 4rg + j
#pragma unroll
    for (int i = 0; i < TPW; i++) {
        const int q = TPW * wave + i, rg = q % NRG, th = q / NRG;
        const float *a = acc[i];
        float res[4];
        if constexpr (FUSED) {
            float b[16];
#pragma unroll
            for (int v = 0; v < 16; v++) b[v] = __fadd_rn(a[v], __shfl_xor(a[v], 32));   // a_s + a_(s+4)
#pragma unroll
            for (int j = 0; j < 4; j++)
                res[j] = __fadd_rn(__fadd_rn(b[4 * j], b[4 * j + 1]), __fadd_rn(b[4 * j + 2], b[4 * j + 3]));
        } else {
#pragma unroll
            for (int j = 0; j < 4; j++) res[j] = a[j];
        }
        const int64_t t = t0 + 32 * th + col;
        const int64_t row = r0 + 4 * rg;
        if (h == 0 && t < m) {
#pragma unroll
            for (int j = 0; j < 4; j++)
                if (row + j < n) __builtin_nontemporal_store(res[j], &y[t * n + row + j]);
        }
    }
}

hipError_t launch_gemm(int type, const uint8_t *w, int64_t n, int64_t k, const uint8_t *xq, int64_t m,
                       float *y, int fused, hipStream_t s) {
    if (type == 8) {
        const int nb = (int)(k / QK8_0);
        // 32 x 32 tiles: eight MFMA tiles, one per wave (measured against
        // 32 x 64 and 16 x 64 at M = 64..2048: 14.7 / 18.2 / 15.5 us at
        // M = 512, N = K = 1024)
        const dim3 grid((unsigned)((n + 31) / 32), (unsigned)((m + 31) / 32));
        if (fused) hipLaunchKernelGGL((k_gemm_q80<true, 32, 32>), grid, dim3(512), 0, s, w, n, nb, xq, m, y);
        else hipLaunchKernelGGL((k_gemm_q80<false, 32, 32>), grid, dim3(512), 0, s, w, n, nb, xq, m, y);
        return hipGetLastError();
    }
    const int nb = (int)(k / QK_K);
    if (type == 12 || type == 13) {
        // 128-token tiles once they give at least three quarters of the CUs
        // a workgroup. Q4_K (two workgroups per CU) at N = 3584, K = 1024:
        // faster at 224 to 896 tiles, slower at 112. Q5_K's three planes
        // leave room for one workgroup per CU, so its tiles must fit one
        // round: faster at 224 (14.2 -> 12.7 us), slower at 336 and 896.
        const unsigned mtw = (unsigned)((m + GW_BM - 1) / GW_BM);
        const uint64_t tiles = (uint64_t)((n + 63) / 64) * mtw;
        // Q4_K there: weight rows in registers instead (k_gemm_r), 32-token
        // tiles below 1024 tokens, 64-token tiles from there (N = 3584,
        // K = 1024: M = 512 10.7 against 11.0 us, 1024 15.3 against 16.0,
        // 2048 27.9 against 30.0)
        // Q4_K up to 704 tokens: the super-blocks of a 32 x 32 tile across
        // the waves of one workgroup (k_gemm_ks). N = 3584, K = 1024: M = 64
        // 4.2 against 7.5 us, 128 5.2 / 7.4, 256 6.8 / 9.7, 384 8.7 / 11.4,
        // 512 10.1 / 10.4 (k_gemm_r), 640 12.4 / 13.7; 768 14.7 / 14.1,
        // 1024 18.4 / 15.5, 2048 34 / 29.
        if (type == 12 && m <= 704) {
            // terms in the activations' LDS once the tiles outnumber three
            // workgroups per CU (N = 3584, K = 1024: M = 512 10.1 -> 9.6 us,
            // 256 6.77 -> 6.67; M = 128 keeps the separate arrays, 5.17
            // against 5.24)
            const dim3 grid((unsigned)((n + 31) / 32), (unsigned)((m + 31) / 32));
            const bool share = (uint64_t)grid.x * grid.y > 3 * 256;
#define QK_KS_LAUNCH(F, S) hipLaunchKernelGGL((k_gemm_ks<F, S>), grid, dim3(256), 0, s, w, n, nb, xq, m, y)
            if (fused) { if (share) QK_KS_LAUNCH(true, true); else QK_KS_LAUNCH(true, false); }
            else { if (share) QK_KS_LAUNCH(false, true); else QK_KS_LAUNCH(false, false); }
#undef QK_KS_LAUNCH
            return hipGetLastError();
        }
        if (tiles >= 192 && type == 12) {
            if (m < 1024) {
                const dim3 grid((unsigned)((n + 127) / 128), (unsigned)((m + 31) / 32));
                if (fused) hipLaunchKernelGGL((k_gemm_r<true, 32>), grid, dim3(256), 0, s, w, n, nb, xq, m, y);
                else hipLaunchKernelGGL((k_gemm_r<false, 32>), grid, dim3(256), 0, s, w, n, nb, xq, m, y);
            } else {
                const dim3 grid((unsigned)((n + 127) / 128), (unsigned)((m + 63) / 64));
                if (fused) hipLaunchKernelGGL((k_gemm_r<true, 64>), grid, dim3(256), 0, s, w, n, nb, xq, m, y);
                else hipLaunchKernelGGL((k_gemm_r<false, 64>), grid, dim3(256), 0, s, w, n, nb, xq, m, y);
            }
            return hipGetLastError();
        }
        if (tiles >= 192 && tiles <= 256) {              // Q5_K
            const dim3 grid((unsigned)((n + 63) / 64), mtw);
            if (fused) hipLaunchKernelGGL((k_gemm_w<13, true>), grid, dim3(512), 0, s, w, n, nb, xq, m, y);
            else hipLaunchKernelGGL((k_gemm_w<13, false>), grid, dim3(512), 0, s, w, n, nb, xq, m, y);
            return hipGetLastError();
        }
    }
    // Q6_K up to 512 tokens: super-blocks across waves (k_gemm_ks6). N =
    // 1024, K = 3584: M = 128 13.9 against 22.3 us, 256 13.9 / 22.3, 512
    // 18.4 / 22.4; 1024 37.3 / 33.0.
    if (type == 14 && m <= 512) {
        const dim3 grid((unsigned)((n + 31) / 32), (unsigned)((m + 31) / 32));
        if (m <= 256) {                                // 8 super-blocks a round: 128 / 256 tokens 13.9 us
            if (fused) hipLaunchKernelGGL((k_gemm_ks6<true, 8>), grid, dim3(512), 0, s, w, n, nb, xq, m, y);
            else hipLaunchKernelGGL((k_gemm_ks6<false, 8>), grid, dim3(512), 0, s, w, n, nb, xq, m, y);
        } else {                                       // 4: 512 tokens 18.4 us (21.1 with 8)
            if (fused) hipLaunchKernelGGL((k_gemm_ks6<true, 4>), grid, dim3(256), 0, s, w, n, nb, xq, m, y);
            else hipLaunchKernelGGL((k_gemm_ks6<false, 4>), grid, dim3(256), 0, s, w, n, nb, xq, m, y);
        }
        return hipGetLastError();
    }
    const unsigned mt = (unsigned)((m + GM_BM - 1) / GM_BM);
    // 64-row tiles when they alone give every CU a workgroup, else 32-row
    // tiles (twice the workgroups, k split four ways)
    const bool narrow = (uint64_t)((n + 63) / 64) * mt < 256;
    const dim3 grid64((unsigned)((n + 63) / 64), mt), grid32((unsigned)((n + 31) / 32), mt);
#define QK_GEMM_LAUNCH(T)                                                                                   \
    do {                                                                                                    \
        if (narrow) {                                                                                       \
            if (fused) hipLaunchKernelGGL((k_gemm<T, true, 32>), grid32, dim3(512), 0, s, w, n, nb, xq, m, y); \
            else hipLaunchKernelGGL((k_gemm<T, false, 32>), grid32, dim3(512), 0, s, w, n, nb, xq, m, y);      \
        } else {                                                                                            \
            if (fused) hipLaunchKernelGGL((k_gemm<T, true, 64>), grid64, dim3(512), 0, s, w, n, nb, xq, m, y); \
            else hipLaunchKernelGGL((k_gemm<T, false, 64>), grid64, dim3(512), 0, s, w, n, nb, xq, m, y);      \
        }                                                                                                   \
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
