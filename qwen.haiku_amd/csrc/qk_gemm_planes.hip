// qk_gemm_planes.hip -- chunked-prefill GEMM over K-quant weights repacked
// once into int8 MFMA planes (gfx950).
//
// The native-block GEMM (qk_gemm.hip) re-derives, for every token tile,
// the int8 operands of a weight tile from its 4/5/6-bit quants and 6-bit
// or int8 scales: about half of its vector instructions. Weights are
// immutable after load (slm/slm.h:12-13) and HBM is plentiful, so this
// path does that work once per matrix: k_pack_planes writes each 32-row
// group's super-block as the exact B operands of the MFMAs, and the GEMM
// only loads them.
//
// Planes. Per row and super-block, the weight w_e and its sub-block scale
// fold into one integer v_e (exact):
//   Q4_K / Q5_K: v_e = sc_j * q_e        in [0, 63 * 31]
//   Q6_K:        v_e = sc_s * (u6_e - 32) in [-4064, 4096]
// split as v_e = 128 * hi_e + lo_e with lo_e = v_e & 127 in [0, 127] and
// hi_e = v_e >> 7 (arithmetic) in [-32, 32]: two int8 planes. With
// acc_p = sum_e plane_p[e] * q8_e (one chain of v_mfma_i32_32x32x32_i8 per
// plane, exact in int32),
//   Q4_K / Q5_K: isum            = acc_lo + 128 * acc_hi
//                (simd/quants.h:283-304, 324-349)
//   Q6_K:        isum - 32 * isum_mins = acc_lo + 128 * acc_hi
//                (simd/quants.h:356-399: sum_s sc_s * sum_e (u6_e - 32) q8_e)
// The Q4_K / Q5_K mins sum_j m_j * (bsums[2j] + bsums[2j+1]) is one
// v_mfma_f32_32x32x16_f16 of the sixteen bsums (|bsum| <= 16 * 128 = 2048,
// exact in f16) against the mins, each repeated twice (exact in f16); every
// product and partial sum is an integer below 2^24, so the f32 result is
// exact. The super-block's float term and the running sum then follow the
// reference's rounding sequence exactly as in the GEMV and qk_gemm.hip.
//
// Layout of a chunk (row group g = rows 32g..32g+31, super-block i), at
// wp + (g * nb + i) * chunk bytes:
//   [16 KB]  planes: 16 operands (sub-block s, plane p at (2s + p) * 1024),
//            lane l's 16 bytes at 16 l: row 32g + l % 32, elements
//            32s + 16(l / 32) .. + 15 of the super-block (the lane's k
//            range of a 32x32x32 MFMA, the same for both operands);
//   [1 KB]   (Q4_K / Q5_K) mins operand: lane l's eight f16 at 16 l, the
//            mins of bsums 8(l / 32) .. + 7, i.e. m_{4(l/32) + k/2};
//   [256 B]  per row {f32 d, f32 dmin} (Q6_K: {f32 d, 0}), row r at 8 r.
// Rows past n are zero.
#include "qk_dev.h"
#include "qk_kernels.h"

namespace qk {

typedef int32_t p4i __attribute__((ext_vector_type(4)));
typedef int32_t p16i __attribute__((ext_vector_type(16)));
typedef float p16f __attribute__((ext_vector_type(16)));
typedef _Float16 p8h __attribute__((ext_vector_type(8)));

#define PL_PLANES 16384
#define PL_MINS 1024
#define PL_SCAL 256
#define PL_LD 272                      // LDS row stride of the activation quants (256 + 16)

__host__ __device__ constexpr int pl_chunk(int type) {
    return type == 14 ? PL_PLANES + PL_SCAL : PL_PLANES + PL_MINS + PL_SCAL;
}
__host__ __device__ constexpr int pl_scal_off(int type) { return type == 14 ? PL_PLANES : PL_PLANES + PL_MINS; }

// ---- repacking ---------------------------------------------------------------
// One wave per chunk; lane l: row 32g + l % 32, element half h = l / 32 of
// every sub-block. Byte loads throughout (Q6_K blocks are 2-byte aligned);
// the kernel runs once per matrix.
template <int TYPE>
__global__ __launch_bounds__(64) void k_pack_planes(const uint8_t *__restrict__ w, int64_t n, int nb,
                                                    uint8_t *__restrict__ wp) {
    const int lane = threadIdx.x, col = lane & 31, h = lane >> 5;
    const int64_t g = blockIdx.x;
    const int i = blockIdx.y;
    const int64_t row = g * 32 + col;
    const bool in = row < n;
    uint8_t *ck = wp + (g * nb + i) * (int64_t)pl_chunk(TYPE);
    constexpr int BB = TYPE == 12 ? Q4K_BYTES : (TYPE == 13 ? Q5K_BYTES : Q6K_BYTES);
    const uint8_t *b = w + ((in ? row : 0) * nb + i) * (int64_t)BB;
    auto byte = [&](int o) -> uint32_t { return in ? ld_u8(b + o) : 0u; };
    int32_t sc[8], mn[8];
    if (TYPE != 14) {
        uint32_t s[3];
#pragma unroll
        for (int q = 0; q < 3; q++)
            s[q] = byte(4 + 4 * q) | byte(5 + 4 * q) << 8 | byte(6 + 4 * q) << 16 | byte(7 + 4 * q) << 24;
#pragma unroll
        for (int j = 0; j < 8; j++) scale_min(s[0], s[1], s[2], j, sc[j], mn[j]);
    }
#pragma unroll 1
    for (int sbk = 0; sbk < 8; sbk++) {
        uint32_t lo[4] = {0, 0, 0, 0}, hi[4] = {0, 0, 0, 0};
#pragma unroll
        for (int k = 0; k < 16; k++) {
            const int e = 32 * sbk + 16 * h + k;       // element of the super-block
            int32_t v;
            if (TYPE == 14) {
                const int jh = e >> 7, el = e & 127, qq = el >> 5, l = el & 31;
                const uint32_t nib = (byte(64 * jh + 32 * (qq & 1) + l) >> (4 * (qq >> 1))) & 15u;
                const uint32_t hb = (byte(128 + 32 * jh + l) >> (2 * qq)) & 3u;
                const int32_t scs = (int32_t)(int8_t)byte(192 + (e >> 4));
                v = scs * ((int32_t)(nib | hb << 4) - 32);
            } else {
                const int l = e & 31, c = sbk >> 1, hs = sbk & 1;
                const int qo = TYPE == 12 ? 16 : 48;
                int32_t q = (int32_t)((byte(qo + 32 * c + l) >> (4 * hs)) & 15u);
                if (TYPE == 13) q += 16 * (int32_t)((byte(16 + l) >> sbk) & 1u);
                v = sc[sbk] * q;
            }
            lo[k >> 2] |= (uint32_t)(v & 127) << (8 * (k & 3));
            hi[k >> 2] |= ((uint32_t)(v >> 7) & 0xffu) << (8 * (k & 3));
        }
        *(QK_GLOBAL uint4 *)(ck + (2 * sbk) * 1024 + 16 * lane) = make_uint4(lo[0], lo[1], lo[2], lo[3]);
        *(QK_GLOBAL uint4 *)(ck + (2 * sbk + 1) * 1024 + 16 * lane) = make_uint4(hi[0], hi[1], hi[2], hi[3]);
    }
    if (TYPE != 14) {
        p8h m8;
#pragma unroll
        for (int k = 0; k < 8; k++) m8[k] = (_Float16)mn[4 * h + (k >> 1)];
        *(QK_GLOBAL p8h *)(ck + PL_PLANES + 16 * lane) = m8;
    }
    if (h == 0) {
        float d, dm;
        if (TYPE == 14) {
            d = h2f(byte(208) | byte(209) << 8);
            dm = 0.0f;
        } else {
            d = h2f(byte(0) | byte(1) << 8);
            dm = h2f(byte(2) | byte(3) << 8);
        }
        *(QK_GLOBAL float2 *)(ck + pl_scal_off(TYPE) + 8 * col) = make_float2(d, dm);
    }
}

size_t gemm_planes_bytes(int type, int64_t n, int64_t k) {
    if (type != 12 && type != 13 && type != 14) return 0;
    return (size_t)((n + 31) / 32) * (size_t)(k / QK_K) * (size_t)pl_chunk(type);
}

hipError_t launch_pack_planes(int type, const uint8_t *w, int64_t n, int64_t k, uint8_t *wp, hipStream_t s) {
    const int nb = (int)(k / QK_K);
    const dim3 grid((unsigned)((n + 31) / 32), (unsigned)nb);
    switch (type) {
        case 12: hipLaunchKernelGGL(k_pack_planes<12>, grid, dim3(64), 0, s, w, n, nb, wp); break;
        case 13: hipLaunchKernelGGL(k_pack_planes<13>, grid, dim3(64), 0, s, w, n, nb, wp); break;
        case 14: hipLaunchKernelGGL(k_pack_planes<14>, grid, dim3(64), 0, s, w, n, nb, wp); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// ---- the GEMM ------------------------------------------------------------------

__device__ __forceinline__ void pl_barrier() {     // LDS-only workgroup barrier (global loads stay in flight)
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Output element v (0..15) of a lane in a 32x32 MFMA tile: column (weight
// row) = lane % 32, row (token) = 8*(v/4) + 4*(lane/32) + v%4.
__device__ __forceinline__ int pl_tok(int v, int h) { return 8 * (v >> 2) + 4 * h + (v & 3); }

// A 256-thread workgroup owns 4 row groups (wave w: rows 32(4 bx + w) ..)
// x 32 TT tokens and walks the super-blocks in order. The tokens' Q8_K
// quants (and, for Q4_K / Q5_K, their bsums in f16), and d, are staged in
// LDS, double-buffered: during super-block i the workgroup stores i + 1
// (loaded into registers one step earlier) into the other buffer, so one
// barrier per super-block suffices. Each wave holds its chunk's 16 plane
// operands in registers and reloads operand pair s for super-block i + 1
// as soon as super-block i's last MFMA on it has issued; the TT token
// tiles' products run sub-block by sub-block, then their float terms.
// (Issuing tile j + 1's products beside tile j's terms, software-
// pipelined across super-blocks, measured the same and spilled.)
template <int TYPE, bool FUSED, int TT>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2)))
void k_gemm_planes(const uint8_t *__restrict__ wp, int64_t n, int nb, const uint8_t *__restrict__ xq, int64_t m,
                   float *__restrict__ y) {
    constexpr bool KQ = TYPE != 14;
    constexpr int T = 32 * TT;
    constexpr int CH = pl_chunk(TYPE);
    __shared__ __attribute__((aligned(16))) int8_t sa[2][T][PL_LD];
    __shared__ __attribute__((aligned(16))) _Float16 sbs[2][KQ ? T : 1][16];
    __shared__ __attribute__((aligned(16))) float syd[2][T];
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int col = lane & 31, h = lane >> 5;
    const int64_t ngroups = (n + 31) / 32;
    const int64_t g = (int64_t)blockIdx.x * 4 + wave;
    const bool live = g < ngroups;                     // wave-uniform
    const int64_t t0 = (int64_t)blockIdx.y * T;
    const int mrows = (m - t0 < T) ? (int)(m - t0) : T;
    const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t *>(xq + t0 * nb * Q8K_BYTES), 0, mrows * nb * Q8K_BYTES, 0x00020000);
    // activations: thread t stages eighth e = t % 8 (32 quants, bsums 2e
    // and 2e + 1) of tokens t / 8 + 32 jj
    const int at = tid >> 3, ae = tid & 7;
    struct A8 { uint4 q0, q1; uint32_t bp, d; } ar[TT];
    auto load_a = [&](int i) {
#pragma unroll
        for (int jj = 0; jj < TT; jj++) {
            const int o = (at + 32 * jj) * nb * Q8K_BYTES + i * Q8K_BYTES;
            ar[jj].q0 = bl128(xr, o + 4 + 32 * ae);
            ar[jj].q1 = bl128(xr, o + 20 + 32 * ae);
            if (KQ) ar[jj].bp = bl32(xr, o + 260 + 4 * ae);
            ar[jj].d = bl32(xr, o);
        }
    };
    auto store_a = [&](int buf) {
#pragma unroll
        for (int jj = 0; jj < TT; jj++) {
            const int t = at + 32 * jj;
            *(QK_LDS uint4 *)&sa[buf][t][32 * ae] = ar[jj].q0;
            *(QK_LDS uint4 *)&sa[buf][t][32 * ae + 16] = ar[jj].q1;
            if (KQ) {
                typedef _Float16 h2 __attribute__((ext_vector_type(2)));
                const h2 v = {(_Float16)(int16_t)(ar[jj].bp & 0xffffu), (_Float16)(int16_t)(ar[jj].bp >> 16)};
                *(QK_LDS h2 *)&sbs[buf][t][2 * ae] = v;
            }
            syd[buf][t] = __uint_as_float(ar[jj].d);   // the token's eight threads store the same d
        }
    };
    // this wave's chunk operands, through a buffer resource over its row
    // group's chunks: lane offset 16 l in a VGPR, the operand's offset in
    // an SGPR
    const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t *>(wp + (live ? g : 0) * nb * (int64_t)CH), 0, nb * CH, 0x00020000);
    // operand pair s is reloaded for super-block i + 1 right after super-
    // block i's last MFMA on it
    p4i bq[16];
    p8h bmn;
    float bwd = 0.0f, bwdm = 0.0f;
    auto load_pair = [&](int i, int s) {
#pragma unroll
        for (int p = 0; p < 2; p++) {
            const auto v = __builtin_amdgcn_raw_buffer_load_b128(wr, 16 * lane, i * CH + 1024 * (2 * s + p), 0);
            bq[2 * s + p] = p4i{(int)v[0], (int)v[1], (int)v[2], (int)v[3]};
        }
    };
    auto load_side = [&](int i) {
        if (KQ) bmn = __builtin_bit_cast(p8h, __builtin_amdgcn_raw_buffer_load_b128(wr, 16 * lane, i * CH + PL_PLANES, 0));
        const auto sc = __builtin_amdgcn_raw_buffer_load_b64(wr, 8 * col, i * CH + pl_scal_off(TYPE), 0);
        bwd = __uint_as_float(sc[0]);
        bwdm = __uint_as_float(sc[1]);
    };
    float sum[TT][16];
#pragma unroll
    for (int j = 0; j < TT; j++)
#pragma unroll
        for (int v = 0; v < 16; v++) sum[j][v] = 0.0f;
    const p16i zero = {0};
    const p16f zerof = {0.0f};
    if (live) {
#pragma unroll
        for (int s = 0; s < 8; s++) load_pair(0, s);
        load_side(0);
    }
    load_a(0);
    store_a(0);
    if (nb > 1) load_a(1);
    pl_barrier();
    for (int i = 0; i < nb; i++) {
        const int cur = i & 1;
        if (i + 1 < nb) {                              // A(i + 1) into the other buffer
            store_a(cur ^ 1);
            if (i + 2 < nb) load_a(i + 2);
        }
        if (live) {
            const float wd = bwd, wdm = bwdm;
            p16f mf[TT];
            if (KQ) {
#pragma unroll
                for (int j = 0; j < TT; j++) {
                    const p8h amv = *(const QK_LDS p8h *)&sbs[cur][32 * j + col][8 * h];
                    mf[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(amv, bmn, zerof, 0, 0, 0);
                }
            }
            load_side(i + 1);                          // past the last super-block: reads zeros
            p16i a0[TT], a1[TT];
#pragma unroll
            for (int j = 0; j < TT; j++) a0[j] = a1[j] = zero;
#pragma unroll
            for (int s = 0; s < 8; s++) {
                p4i av[TT];
#pragma unroll
                for (int j = 0; j < TT; j++) av[j] = *(const QK_LDS p4i *)&sa[cur][32 * j + col][32 * s + 16 * h];
#pragma unroll
                for (int j = 0; j < TT; j++) {
                    a0[j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(av[j], bq[2 * s], a0[j], 0, 0, 0);
                    a1[j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(av[j], bq[2 * s + 1], a1[j], 0, 0, 0);
                }
                load_pair(i + 1, s);
            }
#pragma unroll
            for (int j = 0; j < TT; j++) {
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    const float4 y4 = *(const QK_LDS float4 *)&syd[cur][32 * j + 8 * q + 4 * h];
                    const float yv[4] = {y4.x, y4.y, y4.z, y4.w};
#pragma unroll
                    for (int r = 0; r < 4; r++) {
                        const int v = 4 * q + r;
                        const float yd = yv[r];
                        const int32_t is = a0[j][v] + 128 * a1[j][v];
                        float term;
                        if (KQ) {
                            const float d = __fmul_rn(yd, wd);
                            const float dmin = __fmul_rn(yd, wdm);
                            const float pm = __fmul_rn(dmin, mf[j][v]);
                            term = FUSED ? __builtin_fmaf(d, (float)is, -pm) : __fsub_rn(__fmul_rn(d, (float)is), pm);
                        } else {
                            term = __fmul_rn(__fmul_rn(wd, yd), (float)is);
                        }
                        sum[j][v] = __fadd_rn(sum[j][v], term);
                    }
                }
            }
        }
        pl_barrier();                                  // buffer cur read by every wave; cur ^ 1 stored
    }
    if (live) {
        const int64_t row = g * 32 + col;
        if (row < n) {
#pragma unroll
            for (int j = 0; j < TT; j++)
#pragma unroll
                for (int v = 0; v < 16; v++) {
                    const int64_t t = t0 + 32 * j + pl_tok(v, h);
                    if (t < m) __builtin_nontemporal_store(FUSED ? bcast8(sum[j][v]) : sum[j][v], &y[t * n + row]);
                }
        }
    }
}

// Super-blocks across waves (short prompts, or few row groups): a
// workgroup of S waves owns one 32-token x 32-row tile; in round r wave w
// computes super-block S r + w from its chunk, straight from memory, and
// writes its 16 terms per lane to LDS; then wave w adds outputs
// (16 / S) w .. of every lane, the round's terms in super-block order, to
// the running sums (which start at +0.0, so the first term enters
// exactly): the reference's sequential `sum += term`. The round's
// activations are staged by all threads.
template <int TYPE, bool FUSED, int S, bool PF>
__global__ __launch_bounds__(64 * S) void k_gemm_planes_ks(const uint8_t *__restrict__ wp, int64_t n, int nb,
                                                        const uint8_t *__restrict__ xq, int64_t m,
                                                        float *__restrict__ y) {
    constexpr bool KQ = TYPE != 14;
    constexpr int CH = pl_chunk(TYPE);
    static_assert(S == 4, "one staging pass covers four super-blocks");
    constexpr int VW = 16 / S;                         // outputs per lane each wave adds up
    __shared__ __attribute__((aligned(16))) int8_t sa[S][32][PL_LD];
    __shared__ __attribute__((aligned(16))) float st[S][16][64];    // the waves' terms, [wave][v][lane]
    __shared__ __attribute__((aligned(16))) _Float16 sbs[KQ ? S : 1][32][16];
    __shared__ __attribute__((aligned(16))) float syd[S][32];
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int col = lane & 31, h = lane >> 5;
    const int64_t g = blockIdx.x, t0 = (int64_t)blockIdx.y * 32;
    const int mrows = (m - t0 < 32) ? (int)(m - t0) : 32;
    const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t *>(xq + t0 * nb * Q8K_BYTES), 0, mrows * nb * Q8K_BYTES, 0x00020000);
    const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t *>(wp + g * nb * (int64_t)CH), 0, nb * CH, 0x00020000);
    // staging: thread t stages eighth e = t % 8 of token t / 8 for the
    // round's four super-blocks
    const int at = tid >> 3, ae = tid & 7;
    float sum[VW];
#pragma unroll
    for (int b = 0; b < VW; b++) sum[b] = 0.0f;
    const p16i zero = {0};
    const p16f zerof = {0.0f};
    // PF (one workgroup per CU, the rounds latency-bound): a round's
    // operands are loaded during the round before, the activations once the
    // previous ones are staged, this wave's planes once the previous MFMAs
    // have read theirs (172 VGPRs for Q6_K). Else at the start of their
    // round. Past the last super-block the planes read zeros and the
    // activations repeat the last block.
    struct A8 { uint4 q0, q1; uint32_t bp, d; };
    struct Ops { p4i bq[16]; p8h bmn; uint32_t scw[2]; A8 ar[4]; };
    auto load_w = [&](Ops &o, int r) {
        const int sb = r + wave;
#pragma unroll
        for (int q = 0; q < 16; q++) {
            const auto v = __builtin_amdgcn_raw_buffer_load_b128(wr, 16 * lane, sb * CH + 1024 * q, 0);
            o.bq[q] = p4i{(int)v[0], (int)v[1], (int)v[2], (int)v[3]};
        }
        if (KQ) o.bmn = __builtin_bit_cast(p8h, __builtin_amdgcn_raw_buffer_load_b128(wr, 16 * lane, sb * CH + PL_PLANES, 0));
        const auto sc = __builtin_amdgcn_raw_buffer_load_b64(wr, 8 * col, sb * CH + pl_scal_off(TYPE), 0);
        o.scw[0] = sc[0], o.scw[1] = sc[1];
    };
    auto load_a = [&](Ops &o, int r) {
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const int sq = r + q;
            const int of = at * nb * Q8K_BYTES + (sq < nb ? sq : nb - 1) * Q8K_BYTES;
            o.ar[q].q0 = bl128(xr, of + 4 + 32 * ae);
            o.ar[q].q1 = bl128(xr, of + 20 + 32 * ae);
            if (KQ) o.ar[q].bp = bl32(xr, of + 260 + 4 * ae);
            o.ar[q].d = bl32(xr, of);
        }
    };
    // round r from the operands in o, which it reloads for round r + S
    auto round = [&](Ops &o, int r) __attribute__((always_inline)) {
        const int sb = r + wave;
        const bool act = sb < nb;                      // wave-uniform
        const float wd = __uint_as_float(o.scw[0]), wdm = __uint_as_float(o.scw[1]);
        if (r > 0) pl_barrier();                       // the previous round's reads of st done
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const int qq = q;
            *(QK_LDS uint4 *)&sa[qq][at][32 * ae] = o.ar[q].q0;
            *(QK_LDS uint4 *)&sa[qq][at][32 * ae + 16] = o.ar[q].q1;
            if (KQ) {
                typedef _Float16 h2 __attribute__((ext_vector_type(2)));
                const h2 v = {(_Float16)(int16_t)(o.ar[q].bp & 0xffffu), (_Float16)(int16_t)(o.ar[q].bp >> 16)};
                *(QK_LDS h2 *)&sbs[qq][at][2 * ae] = v;
            }
            syd[qq][at] = __uint_as_float(o.ar[q].d); // the token's eight threads store the same d
        }
        const bool more = r + S < nb;                  // uniform
        if (more) load_a(o, r + S);
        pl_barrier();
        p16i a0 = zero, a1 = zero;
        p16f mf = zerof;
        float yv[16];
        if (act) {
            if (KQ) {
                const p8h amv = *(const QK_LDS p8h *)&sbs[wave][col][8 * h];
                mf = __builtin_amdgcn_mfma_f32_32x32x16_f16(amv, o.bmn, zerof, 0, 0, 0);
            }
#pragma unroll
            for (int s = 0; s < 8; s++) {
                const p4i av = *(const QK_LDS p4i *)&sa[wave][col][32 * s + 16 * h];
                a0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(av, o.bq[2 * s], a0, 0, 0, 0);
                a1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(av, o.bq[2 * s + 1], a1, 0, 0, 0);
            }
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const float4 y4 = *(const QK_LDS float4 *)&syd[wave][8 * q + 4 * h];
                yv[4 * q] = y4.x, yv[4 * q + 1] = y4.y, yv[4 * q + 2] = y4.z, yv[4 * q + 3] = y4.w;
            }
        }
        if (more) load_w(o, r + S);
        if (act) {
#pragma unroll
            for (int v = 0; v < 16; v++) {
                const float yd = yv[v];
                const int32_t is = a0[v] + 128 * a1[v];
                float term;
                if (KQ) {
                    const float d = __fmul_rn(yd, wd);
                    const float dmin = __fmul_rn(yd, wdm);
                    const float pm = __fmul_rn(dmin, mf[v]);
                    term = FUSED ? __builtin_fmaf(d, (float)is, -pm) : __fsub_rn(__fmul_rn(d, (float)is), pm);
                } else {
                    term = __fmul_rn(__fmul_rn(wd, yd), (float)is);
                }
                st[wave][v][lane] = term;
            }
        }
        pl_barrier();
#pragma unroll
        for (int q = 0; q < S; q++) {
            if (r + q >= nb) break;                    // uniform
#pragma unroll
            for (int b = 0; b < VW; b++) sum[b] = __fadd_rn(sum[b], st[q][VW * wave + b][lane]);
        }
    };
    if constexpr (PF) {
        Ops o;
        load_w(o, 0);
        load_a(o, 0);
        for (int r = 0; r < nb; r += S) round(o, r);
    } else {
        for (int r = 0; r < nb; r += S) {
            const int sb = r + wave;
            const bool act = sb < nb;                      // wave-uniform
            // this wave's operands (past the last super-block: zeros)
            p4i bq[16];
            p8h bmn;
    #pragma unroll
            for (int q = 0; q < 16; q++) {
                const auto v = __builtin_amdgcn_raw_buffer_load_b128(wr, 16 * lane, sb * CH + 1024 * q, 0);
                bq[q] = p4i{(int)v[0], (int)v[1], (int)v[2], (int)v[3]};
            }
            if (KQ) bmn = __builtin_bit_cast(p8h, __builtin_amdgcn_raw_buffer_load_b128(wr, 16 * lane, sb * CH + PL_PLANES, 0));
            const auto sc = __builtin_amdgcn_raw_buffer_load_b64(wr, 8 * col, sb * CH + pl_scal_off(TYPE), 0);
            const float wd = __uint_as_float(sc[0]), wdm = __uint_as_float(sc[1]);
            // the round's activations
            struct A8 { uint4 q0, q1; uint32_t bp, d; } ar[4];
    #pragma unroll
            for (int q = 0; q < 4; q++) {
                const int sq = r + q;
                const int o = at * nb * Q8K_BYTES + (sq < nb ? sq : nb - 1) * Q8K_BYTES;
                ar[q].q0 = bl128(xr, o + 4 + 32 * ae);
                ar[q].q1 = bl128(xr, o + 20 + 32 * ae);
                if (KQ) ar[q].bp = bl32(xr, o + 260 + 4 * ae);
                ar[q].d = bl32(xr, o);
            }
            if (r > 0) pl_barrier();                       // the previous round's reads of st done
    #pragma unroll
            for (int q = 0; q < 4; q++) {
                const int qq = q;
                *(QK_LDS uint4 *)&sa[qq][at][32 * ae] = ar[q].q0;
                *(QK_LDS uint4 *)&sa[qq][at][32 * ae + 16] = ar[q].q1;
                if (KQ) {
                    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
                    const h2 v = {(_Float16)(int16_t)(ar[q].bp & 0xffffu), (_Float16)(int16_t)(ar[q].bp >> 16)};
                    *(QK_LDS h2 *)&sbs[qq][at][2 * ae] = v;
                }
                syd[qq][at] = __uint_as_float(ar[q].d);   // the token's eight threads store the same d
            }
            pl_barrier();
            p16i a0 = zero, a1 = zero;
            p16f mf = zerof;
            float yv[16];
            if (act) {
                if (KQ) {
                    const p8h amv = *(const QK_LDS p8h *)&sbs[wave][col][8 * h];
                    mf = __builtin_amdgcn_mfma_f32_32x32x16_f16(amv, bmn, zerof, 0, 0, 0);
                }
    #pragma unroll
                for (int s = 0; s < 8; s++) {
                    const p4i av = *(const QK_LDS p4i *)&sa[wave][col][32 * s + 16 * h];
                    a0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(av, bq[2 * s], a0, 0, 0, 0);
                    a1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(av, bq[2 * s + 1], a1, 0, 0, 0);
                }
    #pragma unroll
                for (int q = 0; q < 4; q++) {
                    const float4 y4 = *(const QK_LDS float4 *)&syd[wave][8 * q + 4 * h];
                    yv[4 * q] = y4.x, yv[4 * q + 1] = y4.y, yv[4 * q + 2] = y4.z, yv[4 * q + 3] = y4.w;
                }
            }
            if (act) {
    #pragma unroll
                for (int v = 0; v < 16; v++) {
                    const float yd = yv[v];
                    const int32_t is = a0[v] + 128 * a1[v];
                    float term;
                    if (KQ) {
                        const float d = __fmul_rn(yd, wd);
                        const float dmin = __fmul_rn(yd, wdm);
                        const float pm = __fmul_rn(dmin, mf[v]);
                        term = FUSED ? __builtin_fmaf(d, (float)is, -pm) : __fsub_rn(__fmul_rn(d, (float)is), pm);
                    } else {
                        term = __fmul_rn(__fmul_rn(wd, yd), (float)is);
                    }
                    st[wave][v][lane] = term;
                }
            }
            pl_barrier();
    #pragma unroll
            for (int q = 0; q < S; q++) {
                if (r + q >= nb) break;                    // uniform
    #pragma unroll
                for (int b = 0; b < VW; b++) sum[b] = __fadd_rn(sum[b], st[q][VW * wave + b][lane]);
            }
        }
    }
    const int64_t row = g * 32 + col;
    if (row < n) {
#pragma unroll
        for (int b = 0; b < VW; b++) {
            const int64_t t = t0 + pl_tok(VW * wave + b, h);
            if (t < m) __builtin_nontemporal_store(FUSED ? bcast8(sum[b]) : sum[b], &y[t * n + row]);
        }
    }
}

template <int TYPE>
static void launch_planes(const uint8_t *wp, int64_t n, int nb, const uint8_t *xq, int64_t m, float *y, int fused,
                          bool ks, hipStream_t s) {
    if (ks) {
        // Q6_K: operands a round ahead when the tiles fit one workgroup per
        // CU (1024 x 3584: M = 128 11.3 -> 10.4 us; Q5_K and more tiles
        // were slower with it)
        const dim3 grid((unsigned)((n + 31) / 32), (unsigned)((m + 31) / 32));
        const bool pf = (uint64_t)grid.x * grid.y <= 256;
#define QK_PLKS(F, P) hipLaunchKernelGGL((k_gemm_planes_ks<TYPE, F, 4, P>), grid, dim3(256), 0, s, wp, n, nb, xq, m, y)
        if constexpr (TYPE == 14) {
            if (pf) {
                if (fused) QK_PLKS(true, true);
                else QK_PLKS(false, true);
                return;
            }
        }
        if (fused) QK_PLKS(true, false);
        else QK_PLKS(false, false);
#undef QK_PLKS
    } else {
        const dim3 grid((unsigned)(((n + 31) / 32 + 3) / 4), (unsigned)((m + 63) / 64));
        if (fused) hipLaunchKernelGGL((k_gemm_planes<TYPE, true, 2>), grid, dim3(256), 0, s, wp, n, nb, xq, m, y);
        else hipLaunchKernelGGL((k_gemm_planes<TYPE, false, 2>), grid, dim3(256), 0, s, wp, n, nb, xq, m, y);
    }
}

// Kernel choice by 32 x 32 output tiles (one MI355X, Q5_K / Q6_K shapes of
// config 3 and the model's projections, M = 64 .. 2048): up to 1024 tiles
// the super-blocks run across waves (k_gemm_planes_ks: Q6_K 1024 x 3584
// at M = 512 15.1 us against 22.4 for k_gemm_planes, Q5_K 2048 x 1024 at
// M = 512 8.3 / 12.2); beyond, 64-token tiles walk the super-blocks
// (Q6_K at M = 2048 28.0 / 37.6, Q5_K 2048 x 1024 at M = 1024 11.0 /
// 12.6). One token tile or four per wave, and eight waves per tile, were
// slower everywhere.
hipError_t launch_gemm_planes(int type, const uint8_t *wp, int64_t n, int64_t k, const uint8_t *xq, int64_t m,
                              float *y, int fused, hipStream_t s) {
    const int nb = (int)(k / QK_K);
    const bool ks = (uint64_t)((n + 31) / 32) * (uint64_t)((m + 31) / 32) <= 1024 && (m + 31) / 32 <= 65535;
    switch (type) {
        case 12: launch_planes<12>(wp, n, nb, xq, m, y, fused, ks, s); break;
        case 13: launch_planes<13>(wp, n, nb, xq, m, y, fused, ks, s); break;
        case 14: launch_planes<14>(wp, n, nb, xq, m, y, fused, ks, s); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace qk
