// qk_deltanet.hip -- the chunked Gated DeltaNet prefill (gfx950).
//
// chunked_ssm_step_f32 (slm/chunked.c:287-521) for every head of a layer
// and every chunk of up to 64 tokens, the state of each head carried from
// chunk to chunk as slm_forward_ssm_batch does (slm/qwen.c:772-807).
//
// The reference runs on the host with plain fp32 loops; on x86 each dot
// and each axpy is a sequential chain of separately rounded products and
// sums (no FMA in its build), and its result depends on that order. Here
// every output element is one lane that runs its reduction in exactly the
// reference's order, skipping the zero coefficients the reference skips;
// the parallelism is across outputs, heads and chunks. There are seven
// phases, each reading the previous phases' results from the per-(chunk,
// head) scratch below; phases 1-4 do not depend on the carried state and
// run for a group of chunks at once, one launch each, and phases 5-7 run
// chunk after chunk inside one launch (this file is built with
// -ffp-contract=off; the only fused multiply-adds are inside qk_expf):
//
//   1 cumulative gate, exps, decay mask; K*beta, V*beta, K*beta*exp(gcs),
//     Q*exp(gcs)
//   2 KK^T and KQ^T scaled by the decay (tiles staged in LDS)
//   3 forward substitution of the unit lower system, one lane per column
//   4 attn @ V*beta, attn @ K*beta*exp(gcs)
//   5 the carried state against Q*exp(gcs) and against the decayed keys;
//     v_new
//   6 the intra-chunk attention on v_new; the output rows
//   7 state := state * exp(g_last) + (K * exp(g_last - gcs))^T v_new
#include "qk_dev.h"
#include "qk_expf.h"
#include "qk_kernels.h"

namespace qk {

constexpr int DN_C = 64;                               // chunk size (CHUNK_SIZE)
constexpr int DN_D = 128;                              // largest head dim handled

// Scratch of one group of chunks (floats), one slot per (chunk, head).
struct DnScratch {
    float *gv;      // [H][3*64 + 1]: gcs | exp(gcs) | exp(glast - gcs) | exp(glast)
    float *dm;      // [H][64][64] decay mask
    float *kb;      // [H][64][kd] K * beta
    float *vb;      // [H][64][vd] V * beta
    float *kbg;     // [H][64][kd] K * beta * exp(gcs)
    float *qg;      // [H][64][kd] Q * exp(gcs)
    float *kkd;     // [H][64][64] strictly lower (K_j . Kbeta_i) * decay
    float *akq;     // [H][64][64] lower (K_j . Q_i) * decay
    float *attn;    // [H][64][64] solved, unit diagonal
    float *veff;    // [H][64][vd]
    float *kcd;     // [H][64][kd]
};

struct DnArgs {
    const float *q, *k, *v, *g, *beta;   // [n_tok][H][...]
    float *state;                        // [H][kd][vd]
    float *out;                          // [n_tok][H][vd]
    int64_t n_tok;                       // tokens of the call
    int64_t g0;                          // first chunk of the group in flight
    int32_t H, kd, vd;
};

// A scratch slot is one (chunk of the group, head): slot = c * H + h.
struct DnChunk {
    int slot, h, n;                      // slot, head, tokens of the chunk (1..64)
    int64_t c0;                          // first token of the chunk
};

__device__ __forceinline__ DnChunk dn_chunk(const DnArgs &a, int slot) {
    DnChunk ck;
    ck.slot = slot;
    ck.h = slot % a.H;
    ck.c0 = (a.g0 + slot / a.H) * DN_C;
    const int64_t rest = a.n_tok - ck.c0;
    ck.n = rest < DN_C ? (int)rest : DN_C;
    return ck;
}

__device__ __forceinline__ const float *row_of(const float *base, const DnArgs &a, int64_t c0, int t, int h,
                                               int dim) {
    return base + ((c0 + t) * a.H + h) * (int64_t)dim;
}

// 1. grid (DN_PREP parts, slots): every part rebuilds the cumulative gate
// of its slot (the g row staged in LDS by 64 lanes at once, then the serial
// sum) and takes every DN_PREP-th slice of the elementwise work; part 0
// writes the gate vectors.
constexpr int DN_PREP = 8;

__global__ __launch_bounds__(256) void k_dn_prep(DnArgs a, DnScratch s) {
    const DnChunk ck = dn_chunk(a, blockIdx.y);
    const int h = ck.h, part = blockIdx.x, n = ck.n, kd = a.kd, vd = a.vd;
    __shared__ float gcs[DN_C], gex[DN_C];
    float *gv = s.gv + (int64_t)ck.slot * (3 * DN_C + 1);
    if (threadIdx.x < n) gcs[threadIdx.x] = a.g[(ck.c0 + threadIdx.x) * a.H + h];
    __syncthreads();
    if (threadIdx.x == 0) {
        float run = 0.0f;
        for (int t = 0; t < n; t++) {
            run = __fadd_rn(run, gcs[t]);
            gcs[t] = run;
        }
    }
    __syncthreads();
    const float glast = gcs[n - 1];
    for (int t = threadIdx.x; t < n; t += 256) {
        gex[t] = qk_expf(gcs[t]);
        if (part == 0) {
            gv[t] = gcs[t];
            gv[DN_C + t] = gex[t];
            gv[2 * DN_C + t] = qk_expf(__fsub_rn(glast, gcs[t]));
        }
    }
    if (part == 0 && threadIdx.x == 0) gv[3 * DN_C] = qk_expf(glast);
    __syncthreads();
    const int first = part * 256 + threadIdx.x, stride = 256 * DN_PREP;
    float *dm = s.dm + (int64_t)ck.slot * DN_C * DN_C;
    for (int p = first; p < n * n; p += stride) {
        const int i = p / n, j = p % n;
        dm[i * DN_C + j] = i > j ? qk_expf(__fsub_rn(gcs[i], gcs[j])) : 0.0f;
    }
    const int64_t ho = (int64_t)ck.slot * DN_C;
    // the rows in rounds of four elements per thread, every load of a
    // round in flight before its products (64 x 128 elements: one round)
    for (int p0 = first; p0 < n * kd; p0 += 4 * stride) {
        float kv[4], qv[4], bv[4];
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const int p = p0 + u * stride, t = p / kd, d = p % kd;
            const bool in = p < n * kd;
            kv[u] = in ? row_of(a.k, a, ck.c0, t, h, kd)[d] : 0.0f;
            qv[u] = in ? row_of(a.q, a, ck.c0, t, h, kd)[d] : 0.0f;
            bv[u] = in ? a.beta[(ck.c0 + t) * a.H + h] : 0.0f;
        }
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const int p = p0 + u * stride, t = p / kd, d = p % kd;
            if (p < n * kd) {
                const float kbv = __fmul_rn(kv[u], bv[u]);
                const float ge = gex[t];
                s.kb[(ho + t) * kd + d] = kbv;
                s.kbg[(ho + t) * kd + d] = __fmul_rn(kbv, ge);
                s.qg[(ho + t) * kd + d] = __fmul_rn(ge, qv[u]);
            }
        }
    }
    for (int p0 = first; p0 < n * vd; p0 += 4 * stride) {
        float vv[4], bv[4];
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const int p = p0 + u * stride, t = p / vd, e = p % vd;
            const bool in = p < n * vd;
            vv[u] = in ? row_of(a.v, a, ck.c0, t, h, vd)[e] : 0.0f;
            bv[u] = in ? a.beta[(ck.c0 + t) * a.H + h] : 0.0f;
        }
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const int p = p0 + u * stride, t = p / vd, e = p % vd;
            if (p < n * vd) s.vb[(ho + t) * vd + e] = __fmul_rn(vv[u], bv[u]);
        }
    }
}

// 2. grid (4 j-tiles, 4 i-tiles, slots); a 16x16 tile of (query i, key j) per
// workgroup, the 16 K rows of its keys and the 16 Kbeta / Q rows of its
// queries in LDS
__global__ __launch_bounds__(256) void k_dn_dots(DnArgs a, DnScratch s) {
    const DnChunk ck = dn_chunk(a, blockIdx.z);
    const int h = ck.h, n = ck.n, kd = a.kd;
    const int i0 = blockIdx.y * 16, j0 = blockIdx.x * 16;
    if (i0 >= n || j0 >= n) return;                   // whole workgroup: tile outside the chunk
    // tiles above the diagonal still run: they write the zeros the later
    // phases read there (the reference's matrices hold 0.0f above it)
    __shared__ float kj[16][DN_D + 1], kbi[16][DN_D + 1], qi[16][DN_D + 1];   // padded: row r on bank r
    const int64_t ho = (int64_t)ck.slot * DN_C;
    {
        float vk[8], vb[8], vq[8];
#pragma unroll
        for (int u = 0; u < 8; u++) {                  // 8 * 256 = 16 rows of DN_D
            const int p = u * 256 + threadIdx.x, r = p / DN_D, d = p % DN_D;
            const bool jin = d < kd && j0 + r < n, iin = d < kd && i0 + r < n;
            vk[u] = jin ? row_of(a.k, a, ck.c0, j0 + r, h, kd)[d] : 0.0f;
            vb[u] = iin ? s.kb[(ho + i0 + r) * kd + d] : 0.0f;
            vq[u] = iin ? row_of(a.q, a, ck.c0, i0 + r, h, kd)[d] : 0.0f;
        }
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const int p = u * 256 + threadIdx.x, r = p / DN_D, d = p % DN_D;
            kj[r][d] = vk[u];
            kbi[r][d] = vb[u];
            qi[r][d] = vq[u];
        }
    }
    __syncthreads();
    const int i = i0 + (threadIdx.x >> 4), j = j0 + (threadIdx.x & 15);
    if (i >= n || j >= n) return;
    const float *dm = s.dm + (int64_t)ck.slot * DN_C * DN_C;
    float kk = 0.0f, kq = 0.0f;
    if (i > j) {
        float acc = 0.0f;
        for (int d = 0; d < kd; d++) acc = __fadd_rn(acc, __fmul_rn(kj[threadIdx.x & 15][d], kbi[threadIdx.x >> 4][d]));
        kk = __fmul_rn(acc, dm[i * DN_C + j]);
    }
    if (i >= j) {
        float acc = 0.0f;
        for (int d = 0; d < kd; d++) acc = __fadd_rn(acc, __fmul_rn(kj[threadIdx.x & 15][d], qi[threadIdx.x >> 4][d]));
        kq = __fmul_rn(acc, i == j ? 1.0f : dm[i * DN_C + j]);
    }
    s.kkd[(ho + i) * DN_C + j] = kk;
    s.akq[(ho + i) * DN_C + j] = kq;
}

// 3. one wave per slot, lane j solves column j of (I + L) X = -L, L the
// strictly lower kkd (slm/chunked.c:196-213): X[i][j] = (-L[i][j] -
// sum_{t<i} L[i][t] X[t][j]) / 1. The order is right-looking: as soon as
// X[k][j] is known every later row adds its term k, so each row's sum
// still runs t = 0, 1, 2, ... in the reference's order while the
// dependent path is a few operations per row. The sums sit in registers
// (both loops unrolled). LS[k] holds column k of L below the diagonal,
// L[k+1 .. 63][k], from its first element, so row k's broadcast
// coefficients arrive as a few aligned 16-byte reads issued together.
// Dividing by the unit diagonal returns its operand unchanged (a quiet NaN
// included), so the division is left out. Rows and columns past the chunk
// run on stale scratch and are not stored; attn = X below the diagonal,
// 1 on it, 0 above.
__global__ __launch_bounds__(64) void k_dn_solve(DnArgs a, DnScratch s) {
    const DnChunk ck = dn_chunk(a, blockIdx.x);
    const int n = ck.n, j = threadIdx.x;
    __shared__ float L[DN_C][DN_C + 1];                // lane j reads column j: no bank conflicts
    __shared__ float4 LS[DN_C][DN_C / 4];              // LS[k][q] = L[k+1+4q .. k+4+4q][k]
    const int64_t ho = (int64_t)ck.slot * DN_C;
    {   // the whole 64x64 tile, sixteen 16-byte loads in flight per lane
        const float4 *src = reinterpret_cast<const float4 *>(s.kkd + ho * DN_C);
        float4 v[16];
#pragma unroll
        for (int u = 0; u < 16; u++) v[u] = src[u * 64 + j];
        float *ls = &LS[0][0].x;
#pragma unroll
        for (int u = 0; u < 16; u++) {
            const int p = (u * 64 + j) * 4, i = p / DN_C, t = p % DN_C;
            const float e[4] = {v[u].x, v[u].y, v[u].z, v[u].w};
#pragma unroll
            for (int c = 0; c < 4; c++) {
                L[i][t + c] = e[c];
                if (i > t + c) ls[(t + c) * DN_C + (i - t - c - 1)] = e[c];
            }
        }
    }
    __syncthreads();
    float acc[DN_C], xs[DN_C];
#pragma unroll
    for (int i = 0; i < DN_C; i++) acc[i] = 0.0f;
#pragma unroll
    for (int k = 0; k < DN_C; k++) {
        const float x = __fsub_rn(-L[k][j], acc[k]);   // -L is -0 on and above the diagonal
        xs[k] = x;
        constexpr int nq_max = DN_C / 4;
        const int nq = (DN_C - 1 - k + 3) / 4;          // compile-time after unrolling
        float cf[DN_C];
#pragma unroll
        for (int q = 0; q < nq_max; q++) {
            if (q < nq) {
                const float4 c4 = LS[k][q];
                cf[4 * q] = c4.x;
                cf[4 * q + 1] = c4.y;
                cf[4 * q + 2] = c4.z;
                cf[4 * q + 3] = c4.w;
            }
        }
#pragma unroll
        for (int i = k + 1; i < DN_C; i++) acc[i] = __fadd_rn(acc[i], __fmul_rn(cf[i - k - 1], x));
        // keep one row's coefficients live at a time: the updates happen
        // here, and the next row's reads stay below
#pragma unroll
        for (int i = k + 1; i < DN_C; i++) asm volatile("" : "+v"(acc[i]));
        asm volatile("" ::: "memory");
    }
    if (j < n) {
        float *attn = s.attn + ho * DN_C;
#pragma unroll
        for (int k = 0; k < DN_C; k++)
            if (k < n) attn[k * DN_C + j] = j < k ? xs[k] : (j == k ? 1.0f : 0.0f);
    }
}

// Phases 4, 6 and 7 read DN_B operands ahead of the dependent adds: every
// scratch row index below stays under DN_C (rows past the chunk hold stale
// data and meet a zero coefficient), and reads of the caller's arrays stop
// at the chunk's last row.
constexpr int DN_R = 4;                                // rows per lane in phase 4
constexpr int DN_B = 8;                                // loads in flight per chain

// 4. grid (8 row blocks, 2, slots), blocks past the chunk exit: a
// workgroup computes eight rows of attn @ V*beta (y = 0) or
// attn @ K*beta*exp(gcs) (y = 1). The rows of the right-hand matrix up to
// the block's last row and the block's eight attn rows (j-major, so one
// 16-byte read gives a lane its four rows' coefficients) are staged in LDS
// with every load in flight at once; lane (row group, e) then runs four
// rows' chains in the reference's j order from LDS. A zero coefficient
// leaves a chain unchanged (the reference skips it). Columns j below the
// group's first row belong to all four rows; the last few columns are
// gated by j <= i. Rows past the chunk are computed and not stored.
constexpr int DN_RB = 8;                               // rows per workgroup

__global__ __launch_bounds__(256) void k_dn_apply(DnArgs a, DnScratch s) {
    const DnChunk ck = dn_chunk(a, blockIdx.z);
    const int n = ck.n, r0 = blockIdx.x * DN_RB;
    if (r0 >= n) return;                               // whole workgroup: rows past the chunk
    const int w = blockIdx.y ? a.kd : a.vd;
    const int64_t ho = (int64_t)ck.slot * DN_C;
    const float *src = blockIdx.y ? s.kbg + ho * a.kd : s.vb + ho * a.vd;
    float *dst = blockIdx.y ? s.kcd + ho * a.kd : s.veff + ho * a.vd;
    __shared__ float M[DN_C * DN_D];
    __shared__ float4 Ct[DN_C][DN_RB / DN_R];          // Ct[j][g]: rows r0+4g .. r0+4g+3 at column j
    const int rows = r0 + DN_RB < n ? r0 + DN_RB : n;  // right-hand rows 0 .. rows-1
    const int total = rows * w;                        // <= 64 * 128 = 32 * 256
    {
        float v[32];
#pragma unroll
        for (int u = 0; u < 32; u++) {
            const int p = u * 256 + threadIdx.x;
            v[u] = p < total ? src[p] : 0.0f;
        }
        const float *arow = s.attn + (ho + r0) * DN_C;   // rows r0 .. r0+7 <= 63
        const float c0 = arow[threadIdx.x], c1 = arow[256 + threadIdx.x];
#pragma unroll
        for (int u = 0; u < 32; u++) {
            const int p = u * 256 + threadIdx.x;
            if (p < total) M[p] = v[u];
        }
        float *ct = &Ct[0][0].x;
        ct[(threadIdx.x % DN_C) * DN_RB + threadIdx.x / DN_C] = c0;
        ct[(threadIdx.x % DN_C) * DN_RB + 4 + threadIdx.x / DN_C] = c1;
    }
    __syncthreads();
    const int rg = threadIdx.x / w, e = threadIdx.x % w;
    const int i0 = r0 + rg * DN_R;
    if (rg >= DN_RB / DN_R || i0 >= n) return;
    const int last = i0 + DN_R - 1 < n - 1 ? i0 + DN_R - 1 : n - 1;
    float acc[DN_R] = {0.0f, 0.0f, 0.0f, 0.0f};
    auto term = [&](int j, const float4 c, float x, bool gate) __attribute__((always_inline)) {
        const float cf[DN_R] = {c.x, c.y, c.z, c.w};
#pragma unroll
        for (int r = 0; r < DN_R; r++) {
            const float k = (!gate || j <= i0 + r) ? cf[r] : 0.0f;
            acc[r] = k != 0.0f ? __fadd_rn(acc[r], __fmul_rn(k, x)) : acc[r];
        }
    };
    int j0 = 0;
    for (; j0 + DN_B <= i0; j0 += DN_B) {              // j < i0: a term of every row of the group
        float xv[DN_B];
        float4 c4[DN_B];
#pragma unroll
        for (int u = 0; u < DN_B; u++) {
            xv[u] = M[(j0 + u) * w + e];
            c4[u] = Ct[j0 + u][rg];
        }
#pragma unroll
        for (int u = 0; u < DN_B; u++) term(j0 + u, c4[u], xv[u], false);
    }
    for (int j = j0; j <= last; j++) term(j, Ct[j][rg], M[j * w + e], true);
#pragma unroll
    for (int r = 0; r < DN_R; r++)
        if (i0 + r <= last) dst[(i0 + r) * w + e] = acc[r];
}

// 5-7 for every chunk of the group in one launch. Each of the three is
// local to a column e of the state: v_new[., e], the output column e and
// the new state column e read only the state column e and per-chunk rows
// every column shares. So a workgroup owns DN_E columns of one head, keeps
// them in LDS and walks the group's chunks in order: grid
// (ceil(vd / DN_E), H), no workgroup waits for another. A chunk's shared
// rows (Q*exp(gcs), the decayed keys, K, the KQ^T decay rows and the gate
// factors) go through registers into LDS, rows padded by one float so the
// eight rows a wave reads sit in different banks; the next chunk's loads
// are issued before this chunk's chains run. Each element's chains run
// in the reference's order, as phases 5-7 above do.
constexpr int DN_E = 8;                                // state columns per workgroup
constexpr int DN_RS = DN_D + 1;                        // padded LDS row of DN_D floats
constexpr int DN_CS = DN_C + 1;                        // padded LDS row of DN_C floats

// Lane (t, e) runs both chains of phase 5 and, over one loop, the output
// chain of (t, e) and the state chains of (t, e) and (t + 64, e).
__global__ __launch_bounds__(512) void k_dn_carry(DnArgs a, DnScratch s, int gc) {
    constexpr int PR = DN_C * DN_D / 512, PA = DN_C * DN_C / 512;   // row / KQ^T elements per lane
    __shared__ float Qs[DN_C * DN_RS], Ks[DN_C * DN_RS], Kr[DN_C * DN_RS], As[DN_C * DN_CS];
    __shared__ float S[DN_D][DN_E], vn[DN_C][DN_E], gf[DN_C + 1];
    const int h = blockIdx.y, e0 = blockIdx.x * DN_E, kd = a.kd, vd = a.vd;
    const int tid = threadIdx.x, el = tid % DN_E, e = e0 + el, t = tid / DN_E;
    const bool col = e < vd;
    float *st = a.state + (int64_t)h * kd * vd;
    for (int p = tid; p < DN_D * DN_E; p += 512) {
        const int d = p / DN_E, c = p % DN_E;
        S[d][c] = d < kd && e0 + c < vd ? st[(int64_t)d * vd + e0 + c] : 0.0f;
    }
    for (int c = 0; c < gc; c++) {
        const DnChunk ck = dn_chunk(a, c * a.H + h);
        const int n = ck.n;
        const int64_t ho = (int64_t)ck.slot * DN_C;
        // the chunk's shared rows: every load in flight, then into LDS
        float rq[PR], rc[PR], rk[PR], ra[PA], rg;
#pragma unroll
        for (int u = 0; u < PR; u++) {
            const int p = tid + 512 * u, tt = p / kd, d = p - tt * kd;
            const bool in = tt < n;
            rq[u] = in ? s.qg[(ho + tt) * kd + d] : 0.0f;
            rc[u] = in ? s.kcd[(ho + tt) * kd + d] : 0.0f;
            rk[u] = in ? row_of(a.k, a, ck.c0, tt, h, kd)[d] : 0.0f;
        }
#pragma unroll
        for (int u = 0; u < PA; u++) {
            const int p = tid + 512 * u;
            ra[u] = p / DN_C < n ? s.akq[ho * DN_C + p] : 0.0f;
        }
        // exp(glast - gcs[t]) for t < 64, exp(glast) at 64
        rg = tid <= DN_C ? s.gv[(int64_t)ck.slot * (3 * DN_C + 1) + 2 * DN_C + tid] : 0.0f;
        __syncthreads();                               // the previous chunk's reads of the rows done
#pragma unroll
        for (int u = 0; u < PR; u++) {
            const int p = tid + 512 * u, tt = p / kd, d = p - tt * kd;
            if (tt < DN_C) {
                Qs[tt * DN_RS + d] = rq[u];
                Ks[tt * DN_RS + d] = rc[u];
                Kr[tt * DN_RS + d] = rk[u];
            }
        }
#pragma unroll
        for (int u = 0; u < PA; u++) {
            const int p = tid + 512 * u;
            As[(p / DN_C) * DN_CS + p % DN_C] = ra[u];
        }
        if (tid <= DN_C) gf[tid] = rg;
        __syncthreads();
        // 5: the chains against the state (Q*exp(gcs) and the decayed
        // keys, skipping zero coefficients as the reference does); v_new
        float ai = 0.0f;
        if (t < n && col) {
            float vp = 0.0f;
            const float *qr = Qs + t * DN_RS, *kr = Ks + t * DN_RS;
#pragma unroll 8
            for (int d = 0; d < kd; d++) {
                const float x = S[d][el], qv = qr[d], kv = kr[d];
                ai = qv != 0.0f ? __fadd_rn(ai, __fmul_rn(qv, x)) : ai;
                vp = kv != 0.0f ? __fadd_rn(vp, __fmul_rn(kv, x)) : vp;
            }
            vn[t][el] = __fsub_rn(s.veff[(ho + t) * vd + e], vp);
        }
        __syncthreads();
        // 6 and 7 over u: the output row's chain (the intra-chunk attention
        // on v_new) and the state's for d = t and t + 64, with
        // K * exp(glast - gcs) rounded as the reference forms it
        const float *kq = As + t * DN_CS;
        const int d0 = t, d1 = t + 64;
        float acc6 = 0.0f, acc0 = 0.0f, acc1 = 0.0f;
#pragma unroll 4
        for (int u = 0; u < n; u++) {
            const float x = vn[u][el], g = gf[u];
            acc6 = __fadd_rn(acc6, __fmul_rn(kq[u], x));
            acc0 = __fadd_rn(acc0, __fmul_rn(__fmul_rn(Kr[u * DN_RS + d0], g), x));
            acc1 = __fadd_rn(acc1, __fmul_rn(__fmul_rn(Kr[u * DN_RS + d1], g), x));
        }
        if (col) {
            if (t < n) a.out[((ck.c0 + t) * a.H + h) * (int64_t)vd + e] = __fadd_rn(ai, acc6);
            if (d0 < kd) S[d0][el] = __fadd_rn(__fmul_rn(S[d0][el], gf[DN_C]), acc0);
            if (d1 < kd) S[d1][el] = __fadd_rn(__fmul_rn(S[d1][el], gf[DN_C]), acc1);
        }
    }
    __syncthreads();
    for (int p = tid; p < DN_D * DN_E; p += 512) {
        const int d = p / DN_E, c = p % DN_E;
        if (d < kd && e0 + c < vd) st[(int64_t)d * vd + e0 + c] = S[d][c];
    }
}

// ---- launcher -----------------------------------------------------------------
// Phases 1-4 read only their chunk's own inputs, so they run for a group
// of chunks at once (one launch per phase over every (chunk, head) slot of
// the group); phases 5-7 carry the state and run chunk after chunk. A
// group holds at most DN_SLOTS slots (one head's slot is about 263 KB of
// scratch at head dims 128), and at least one chunk.
constexpr int DN_SLOTS = 256;

static int dn_group(int32_t H, int64_t n_tok) {
    const int64_t chunks = (n_tok + DN_C - 1) / DN_C;
    const int64_t g = DN_SLOTS / H > 1 ? DN_SLOTS / H : 1;
    return (int)(g < chunks ? g : chunks);
}

size_t deltanet_scratch_bytes(int32_t H, int32_t kd, int32_t vd, int64_t n_tok) {
    const size_t slots = (size_t)dn_group(H, n_tok) * (size_t)H;
    const size_t per = (size_t)(3 * DN_C + 1) + 4 * (size_t)DN_C * DN_C + 4 * (size_t)DN_C * kd +
                       2 * (size_t)DN_C * vd;
    return (per * slots + 11 * 64) * sizeof(float) + 256;   // 11 arrays, each rounded up to 64 floats
}

hipError_t launch_deltanet(const float *q, const float *k, const float *v, const float *g, const float *beta,
                           int64_t n_tok, int32_t H, int32_t kd, int32_t vd, float *state, float *out,
                           void *scratch, hipStream_t st) {
    if (kd > DN_D || vd > DN_D || n_tok < 1 || H < 1) return hipErrorInvalidValue;
    const int G = dn_group(H, n_tok);
    const size_t slots = (size_t)G * (size_t)H;
    float *p = static_cast<float *>(scratch);
    auto take = [&](size_t n_floats) {
        float *r = p;
        p += (n_floats + 63) & ~(size_t)63;            // 256-byte aligned arrays
        return r;
    };
    DnScratch s;
    s.gv = take(slots * (3 * DN_C + 1));
    s.dm = take(slots * DN_C * DN_C);
    s.kkd = take(slots * DN_C * DN_C);
    s.akq = take(slots * DN_C * DN_C);
    s.attn = take(slots * DN_C * DN_C);
    s.kb = take(slots * DN_C * kd);
    s.kbg = take(slots * DN_C * kd);
    s.qg = take(slots * DN_C * kd);
    s.kcd = take(slots * DN_C * kd);
    s.vb = take(slots * DN_C * vd);
    s.veff = take(slots * DN_C * vd);
    const int64_t chunks = (n_tok + DN_C - 1) / DN_C;
    for (int64_t g0 = 0; g0 < chunks; g0 += G) {
        const int gc = (int)(chunks - g0 < G ? chunks - g0 : G);   // chunks in this group
        const unsigned gs = (unsigned)(gc * H);                     // slots in this group
        DnArgs a{q, k, v, g, beta, state, out, n_tok, g0, H, kd, vd};
        hipLaunchKernelGGL(k_dn_prep, dim3(DN_PREP, gs), dim3(256), 0, st, a, s);
        hipLaunchKernelGGL(k_dn_dots, dim3(4, 4, gs), dim3(256), 0, st, a, s);
        hipLaunchKernelGGL(k_dn_solve, dim3(gs), dim3(64), 0, st, a, s);
        hipLaunchKernelGGL(k_dn_apply, dim3(DN_C / DN_RB, 2, gs), dim3(256), 0, st, a, s);
        hipLaunchKernelGGL(k_dn_carry, dim3((vd + DN_E - 1) / DN_E, H), dim3(512), 0, st, a, s, gc);
    }
    return hipGetLastError();
}

}  // namespace qk
