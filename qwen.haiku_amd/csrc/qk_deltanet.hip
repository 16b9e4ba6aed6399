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
// the parallelism is across outputs and heads. A chunk is seven launches,
// one per phase, each reading the previous phases' results from the
// per-head scratch below (this file is built with -ffp-contract=off; the
// only fused multiply-adds are inside qk_expf):
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

// Per-head scratch of one chunk (floats).
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
    float *ainter;  // [H][64][vd]
    float *vnew;    // [H][64][vd]
};

struct DnArgs {
    const float *q, *k, *v, *g, *beta;   // [n_tok][H][...]
    float *state;                        // [H][kd][vd]
    float *out;                          // [n_tok][H][vd]
    int64_t c0;                          // first token of the chunk
    int32_t n, H, kd, vd;
};

__device__ __forceinline__ const float *row_of(const float *base, const DnArgs &a, int t, int h, int dim) {
    return base + ((a.c0 + t) * a.H + h) * (int64_t)dim;
}

// 1. grid (DN_PREP parts, H): every part rebuilds the cumulative gate of
// its head (the g row staged in LDS by 64 lanes at once, then the serial
// sum) and takes every DN_PREP-th slice of the elementwise work; part 0
// writes the gate vectors.
constexpr int DN_PREP = 8;

__global__ __launch_bounds__(256) void k_dn_prep(DnArgs a, DnScratch s) {
    const int h = blockIdx.y, part = blockIdx.x, n = a.n, kd = a.kd, vd = a.vd;
    __shared__ float gcs[DN_C], gex[DN_C];
    float *gv = s.gv + (int64_t)h * (3 * DN_C + 1);
    if (threadIdx.x < n) gcs[threadIdx.x] = a.g[(a.c0 + threadIdx.x) * a.H + h];
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
    float *dm = s.dm + (int64_t)h * DN_C * DN_C;
    for (int p = first; p < n * n; p += stride) {
        const int i = p / n, j = p % n;
        dm[i * DN_C + j] = i > j ? qk_expf(__fsub_rn(gcs[i], gcs[j])) : 0.0f;
    }
    const int64_t ho = (int64_t)h * DN_C;
    for (int p = first; p < n * kd; p += stride) {
        const int t = p / kd, d = p % kd;
        const float b = a.beta[(a.c0 + t) * a.H + h];
        const float kbv = __fmul_rn(row_of(a.k, a, t, h, kd)[d], b);
        const float ge = gex[t];
        s.kb[(ho + t) * kd + d] = kbv;
        s.kbg[(ho + t) * kd + d] = __fmul_rn(kbv, ge);
        s.qg[(ho + t) * kd + d] = __fmul_rn(ge, row_of(a.q, a, t, h, kd)[d]);
    }
    for (int p = first; p < n * vd; p += stride) {
        const int t = p / vd, e = p % vd;
        s.vb[(ho + t) * vd + e] = __fmul_rn(row_of(a.v, a, t, h, vd)[e], a.beta[(a.c0 + t) * a.H + h]);
    }
}

// 2. grid (4 j-tiles, 4 i-tiles, H); a 16x16 tile of (query i, key j) per
// workgroup, the 16 K rows of its keys and the 16 Kbeta / Q rows of its
// queries in LDS
__global__ __launch_bounds__(256) void k_dn_dots(DnArgs a, DnScratch s) {
    const int h = blockIdx.z, n = a.n, kd = a.kd;
    const int i0 = blockIdx.y * 16, j0 = blockIdx.x * 16;
    if (i0 >= n || j0 >= n) return;                   // whole workgroup: tile outside the chunk
    // tiles above the diagonal still run: they write the zeros the later
    // phases read there (the reference's matrices hold 0.0f above it)
    __shared__ float kj[16][DN_D + 1], kbi[16][DN_D + 1], qi[16][DN_D + 1];   // padded: row r on bank r
    const int64_t ho = (int64_t)h * DN_C;
    {
        float vk[8], vb[8], vq[8];
#pragma unroll
        for (int u = 0; u < 8; u++) {                  // 8 * 256 = 16 rows of DN_D
            const int p = u * 256 + threadIdx.x, r = p / DN_D, d = p % DN_D;
            const bool jin = d < kd && j0 + r < n, iin = d < kd && i0 + r < n;
            vk[u] = jin ? row_of(a.k, a, j0 + r, h, kd)[d] : 0.0f;
            vb[u] = iin ? s.kb[(ho + i0 + r) * kd + d] : 0.0f;
            vq[u] = iin ? row_of(a.q, a, i0 + r, h, kd)[d] : 0.0f;
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
    const float *dm = s.dm + (int64_t)h * DN_C * DN_C;
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

// 3. one wave per head, lane j solves column j of (I + L) X = -L, L the
// strictly lower kkd (slm/chunked.c:196-213): X[i][j] = (-L[i][j] -
// sum_{t<i} L[i][t] X[t][j]) / 1. The order is right-looking: as soon as
// X[k][j] is known every later row adds its term k, so each row's sum
// still runs t = 0, 1, 2, ... in the reference's order while the
// dependent path is a few operations per row. The sums sit in registers
// (both loops unrolled) and LT = L transposed in LDS supplies row k's
// broadcast coefficients. Dividing by the unit diagonal returns its
// operand unchanged (a quiet NaN included), so the division is left out.
// Rows and columns past the chunk run on stale scratch and are not
// stored; then attn = X below the diagonal, 1 on it, 0 above.
__global__ __launch_bounds__(64) void k_dn_solve(DnArgs a, DnScratch s) {
    const int h = blockIdx.x, n = a.n, j = threadIdx.x;
    __shared__ float L[DN_C][DN_C + 1];                // lane j reads column j: no bank conflicts
    __shared__ float LT[DN_C][DN_C];                   // LT[t][i] = L[i][t], read as broadcasts
    const int64_t ho = (int64_t)h * DN_C;
    {   // the whole 64x64 tile, sixteen 16-byte loads in flight per lane
        const float4 *src = reinterpret_cast<const float4 *>(s.kkd + ho * DN_C);
        float4 v[16];
#pragma unroll
        for (int u = 0; u < 16; u++) v[u] = src[u * 64 + j];
#pragma unroll
        for (int u = 0; u < 16; u++) {
            const int p = (u * 64 + j) * 4, i = p / DN_C, t = p % DN_C;
            L[i][t] = v[u].x;
            L[i][t + 1] = v[u].y;
            L[i][t + 2] = v[u].z;
            L[i][t + 3] = v[u].w;
            LT[t][i] = v[u].x;
            LT[t + 1][i] = v[u].y;
            LT[t + 2][i] = v[u].z;
            LT[t + 3][i] = v[u].w;
        }
    }
    __syncthreads();
    float *attn = s.attn + ho * DN_C;
    float acc[DN_C];
#pragma unroll
    for (int i = 0; i < DN_C; i++) acc[i] = 0.0f;
#pragma unroll
    for (int k = 0; k < DN_C; k++) {
        const float x = __fsub_rn(-L[k][j], acc[k]);   // -L is -0 on and above the diagonal
        if (k < n && j < n) attn[k * DN_C + j] = j < k ? x : (j == k ? 1.0f : 0.0f);
#pragma unroll
        for (int i = k + 1; i < DN_C; i++) acc[i] = __fadd_rn(acc[i], __fmul_rn(LT[k][i], x));
        // keep one row's coefficients live at a time: the updates happen
        // here, and the next row's loads stay below
#pragma unroll
        for (int i = k + 1; i < DN_C; i++) asm volatile("" : "+v"(acc[i]));
        asm volatile("" ::: "memory");
    }
}

// Phases 4, 6 and 7 read DN_B operands ahead of the dependent adds: every
// scratch row index below stays under DN_C (rows past the chunk hold stale
// data and meet a zero coefficient), and reads of the caller's arrays stop
// at the chunk's last row.
constexpr int DN_R = 4;                                // rows per lane in phase 4
constexpr int DN_B = 8;                                // loads in flight per chain

// 4. grid (ceil(n/8) row blocks, 2, H): a workgroup computes eight rows
// of attn @ V*beta (y = 0) or attn @ K*beta*exp(gcs) (y = 1). The rows of
// the right-hand matrix up to the block's last row and the block's eight
// attn rows are staged in LDS with every load in flight at once; lane
// (row group, e) then runs four rows' chains in the reference's j order
// from LDS. A zero coefficient leaves a chain unchanged (the reference
// skips it), and j runs past a row's end only over zeros.
constexpr int DN_RB = 8;                               // rows per workgroup

__global__ __launch_bounds__(256) void k_dn_apply(DnArgs a, DnScratch s) {
    const int h = blockIdx.z, n = a.n, r0 = blockIdx.x * DN_RB;
    const int w = blockIdx.y ? a.kd : a.vd;
    const int64_t ho = (int64_t)h * DN_C;
    const float *src = blockIdx.y ? s.kbg + ho * a.kd : s.vb + ho * a.vd;
    float *dst = blockIdx.y ? s.kcd + ho * a.kd : s.veff + ho * a.vd;
    __shared__ float M[DN_C * DN_D];
    __shared__ float C[DN_RB][DN_C];
    const int rows = r0 + DN_RB < n ? r0 + DN_RB : n;  // right-hand rows 0 .. rows-1
    const int total = rows * w;                        // <= 64 * 128 = 32 * 256
    {
        float v[32];
#pragma unroll
        for (int u = 0; u < 32; u++) {
            const int p = u * 256 + threadIdx.x;
            v[u] = p < total ? src[p] : 0.0f;
        }
#pragma unroll
        for (int u = 0; u < 32; u++) {
            const int p = u * 256 + threadIdx.x;
            if (p < total) M[p] = v[u];
        }
        const float *arow = s.attn + (ho + r0) * DN_C;   // rows r0 .. r0+7 <= 63
        const float c0 = arow[threadIdx.x], c1 = arow[256 + threadIdx.x];
        (&C[0][0])[threadIdx.x] = c0;
        (&C[0][0])[256 + threadIdx.x] = c1;
    }
    __syncthreads();
    const int rg = threadIdx.x / w, e = threadIdx.x % w;
    const int i0 = r0 + rg * DN_R;
    if (rg >= DN_RB / DN_R || i0 >= n) return;
    const int last = i0 + DN_R - 1 < n - 1 ? i0 + DN_R - 1 : n - 1;
    const float (*cr)[DN_C] = C + rg * DN_R;
    float acc[DN_R] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int j0 = 0; j0 <= last; j0 += DN_B) {         // j0 + DN_B - 1 <= 63
        float xv[DN_B], cf[DN_R][DN_B];
#pragma unroll
        for (int u = 0; u < DN_B; u++) xv[u] = M[(j0 + u) * w + e];
#pragma unroll
        for (int r = 0; r < DN_R; r++)
#pragma unroll
            for (int u = 0; u < DN_B; u++)
                cf[r][u] = (i0 + r <= last && j0 + u <= i0 + r) ? cr[r][j0 + u] : 0.0f;
#pragma unroll
        for (int u = 0; u < DN_B; u++)
#pragma unroll
            for (int r = 0; r < DN_R; r++)
                acc[r] = cf[r][u] != 0.0f ? __fadd_rn(acc[r], __fmul_rn(cf[r][u], xv[u])) : acc[r];
    }
#pragma unroll
    for (int r = 0; r < DN_R; r++)
        if (i0 + r <= last) dst[(i0 + r) * w + e] = acc[r];
}

// 5. grid (ceil(n/4), ceil(vd/64), H): a workgroup takes four rows t and
// 64 columns of the state carried in, both staged in LDS with every load
// in flight at once; wave r runs row t0 + r, lane e its column, the two
// chains (Q*exp(gcs) and the decayed keys against the state) in the
// reference's d order.
constexpr int DN_T = 4;                                // rows per workgroup in phase 5

__global__ __launch_bounds__(256) void k_dn_state_in(DnArgs a, DnScratch s) {
    const int h = blockIdx.z, n = a.n, kd = a.kd, vd = a.vd;
    const int t0 = blockIdx.x * DN_T, e0 = blockIdx.y * 64;
    const int64_t ho = (int64_t)h * DN_C;
    __shared__ float S[DN_D][64];
    __shared__ float Q[DN_T][DN_D], K[DN_T][DN_D];
    {
        const float *st = a.state + (int64_t)h * kd * vd;
        float v[32];
#pragma unroll
        for (int u = 0; u < 32; u++) {                 // 32 * 256 = 128 rows of 64 columns
            const int p = u * 256 + threadIdx.x, d = p >> 6, c = p & 63;
            v[u] = d < kd && e0 + c < vd ? st[(int64_t)d * vd + e0 + c] : 0.0f;
        }
        float cq[2], ck[2];
#pragma unroll
        for (int u = 0; u < 2; u++) {                  // 2 * 256 = DN_T rows of DN_D
            const int p = u * 256 + threadIdx.x, r = p / DN_D, d = p % DN_D;
            const bool in = d < kd && t0 + r < n;
            cq[u] = in ? s.qg[(ho + t0 + r) * kd + d] : 0.0f;
            ck[u] = in ? s.kcd[(ho + t0 + r) * kd + d] : 0.0f;
        }
#pragma unroll
        for (int u = 0; u < 32; u++) {
            const int p = u * 256 + threadIdx.x;
            S[p >> 6][p & 63] = v[u];
        }
#pragma unroll
        for (int u = 0; u < 2; u++) {
            const int p = u * 256 + threadIdx.x;
            Q[p / DN_D][p % DN_D] = cq[u];
            K[p / DN_D][p % DN_D] = ck[u];
        }
    }
    __syncthreads();
    const int r = threadIdx.x >> 6, c = threadIdx.x & 63, t = t0 + r, e = e0 + c;
    if (t >= n || e >= vd) return;
    float ai = 0.0f, vp = 0.0f;
#pragma unroll 8
    for (int d = 0; d < kd; d++) {
        const float x = S[d][c], q = Q[r][d], k = K[r][d];
        ai = q != 0.0f ? __fadd_rn(ai, __fmul_rn(q, x)) : ai;
        vp = k != 0.0f ? __fadd_rn(vp, __fmul_rn(k, x)) : vp;
    }
    s.ainter[(ho + t) * vd + e] = ai;
    s.vnew[(ho + t) * vd + e] = __fsub_rn(s.veff[(ho + t) * vd + e], vp);
}

// 6. grid (n*vd/256, H): lane (t, e), the output row element
__global__ __launch_bounds__(256) void k_dn_out(DnArgs a, DnScratch s) {
    const int h = blockIdx.y, n = a.n, vd = a.vd;
    const int p = blockIdx.x * 256 + threadIdx.x;
    if (p >= n * vd) return;
    const int t = p / vd, e = p % vd;
    const int64_t ho = (int64_t)h * DN_C;
    const float *kq = s.akq + (ho + t) * DN_C;
    const float *vn = s.vnew + ho * vd;
    float acc = 0.0f;
    int u = 0;
    for (; u + DN_B <= n; u += DN_B) {
        float c[DN_B], x[DN_B];
#pragma unroll
        for (int w = 0; w < DN_B; w++) {
            c[w] = kq[u + w];
            x[w] = vn[(u + w) * vd + e];
        }
#pragma unroll
        for (int w = 0; w < DN_B; w++) acc = __fadd_rn(acc, __fmul_rn(c[w], x[w]));
    }
    for (; u < n; u++) acc = __fadd_rn(acc, __fmul_rn(kq[u], vn[u * vd + e]));
    a.out[((a.c0 + t) * a.H + h) * (int64_t)vd + e] = __fadd_rn(s.ainter[(ho + t) * vd + e], acc);
}

// 7. grid (kd*vd/256, H): lane (d, e), the state carried out
__global__ __launch_bounds__(256) void k_dn_state_out(DnArgs a, DnScratch s) {
    const int h = blockIdx.y, n = a.n, kd = a.kd, vd = a.vd;
    const int p = blockIdx.x * 256 + threadIdx.x;
    if (p >= kd * vd) return;
    const int d = p / vd, e = p % vd;
    const int64_t ho = (int64_t)h * DN_C;
    const float *gv = s.gv + (int64_t)h * (3 * DN_C + 1);
    const float *vn = s.vnew + ho * vd;
    float acc = 0.0f;
    int t = 0;
    for (; t + DN_B <= n; t += DN_B) {
        float kg[DN_B], x[DN_B];
#pragma unroll
        for (int w = 0; w < DN_B; w++) {
            kg[w] = __fmul_rn(row_of(a.k, a, t + w, h, kd)[d], gv[2 * DN_C + t + w]);
            x[w] = vn[(t + w) * vd + e];
        }
#pragma unroll
        for (int w = 0; w < DN_B; w++) acc = __fadd_rn(acc, __fmul_rn(kg[w], x[w]));
    }
    for (; t < n; t++) {
        const float kg = __fmul_rn(row_of(a.k, a, t, h, kd)[d], gv[2 * DN_C + t]);
        acc = __fadd_rn(acc, __fmul_rn(kg, vn[t * vd + e]));
    }
    float *st = a.state + (int64_t)h * kd * vd + p;
    *st = __fadd_rn(__fmul_rn(*st, gv[3 * DN_C]), acc);
}

// ---- launcher -----------------------------------------------------------------
size_t deltanet_scratch_bytes(int32_t H, int32_t kd, int32_t vd) {
    const size_t per = (size_t)(3 * DN_C + 1) + 4 * (size_t)DN_C * DN_C + 4 * (size_t)DN_C * kd +
                       4 * (size_t)DN_C * vd;
    return (per * (size_t)H + 13 * 64) * sizeof(float) + 256;   // 13 arrays, each rounded up to 64 floats
}

hipError_t launch_deltanet(const float *q, const float *k, const float *v, const float *g, const float *beta,
                           int64_t n_tok, int32_t H, int32_t kd, int32_t vd, float *state, float *out,
                           void *scratch, hipStream_t st) {
    if (kd > DN_D || vd > DN_D) return hipErrorInvalidValue;
    float *p = static_cast<float *>(scratch);
    auto take = [&](size_t n_floats) {
        float *r = p;
        p += (n_floats + 63) & ~(size_t)63;            // 256-byte aligned arrays
        return r;
    };
    DnScratch s;
    s.gv = take((size_t)H * (3 * DN_C + 1));
    s.dm = take((size_t)H * DN_C * DN_C);
    s.kkd = take((size_t)H * DN_C * DN_C);
    s.akq = take((size_t)H * DN_C * DN_C);
    s.attn = take((size_t)H * DN_C * DN_C);
    s.kb = take((size_t)H * DN_C * kd);
    s.kbg = take((size_t)H * DN_C * kd);
    s.qg = take((size_t)H * DN_C * kd);
    s.kcd = take((size_t)H * DN_C * kd);
    s.vb = take((size_t)H * DN_C * vd);
    s.veff = take((size_t)H * DN_C * vd);
    s.ainter = take((size_t)H * DN_C * vd);
    s.vnew = take((size_t)H * DN_C * vd);
    for (int64_t c0 = 0; c0 < n_tok; c0 += DN_C) {
        DnArgs a{q, k, v, g, beta, state, out, c0, (int32_t)(n_tok - c0 < DN_C ? n_tok - c0 : DN_C), H, kd, vd};
        const int n = a.n;
        hipLaunchKernelGGL(k_dn_prep, dim3(DN_PREP, H), dim3(256), 0, st, a, s);
        hipLaunchKernelGGL(k_dn_dots, dim3(4, 4, H), dim3(256), 0, st, a, s);
        hipLaunchKernelGGL(k_dn_solve, dim3(H), dim3(64), 0, st, a, s);
        hipLaunchKernelGGL(k_dn_apply, dim3((n + DN_RB - 1) / DN_RB, 2, H), dim3(256), 0, st, a, s);
        hipLaunchKernelGGL(k_dn_state_in, dim3((n + DN_T - 1) / DN_T, (vd + 63) / 64, H), dim3(256), 0, st, a, s);
        hipLaunchKernelGGL(k_dn_out, dim3((n * vd + 255) / 256, H), dim3(256), 0, st, a, s);
        hipLaunchKernelGGL(k_dn_state_out, dim3((kd * vd + 255) / 256, H), dim3(256), 0, st, a, s);
    }
    return hipGetLastError();
}

}  // namespace qk
