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

// 1. one workgroup per head
__global__ __launch_bounds__(256) void k_dn_prep(DnArgs a, DnScratch s) {
    const int h = blockIdx.x, n = a.n, kd = a.kd, vd = a.vd;
    __shared__ float gcs[DN_C];
    float *gv = s.gv + (int64_t)h * (3 * DN_C + 1);
    if (threadIdx.x == 0) {
        float run = 0.0f;
        for (int t = 0; t < n; t++) {
            run = __fadd_rn(run, a.g[(a.c0 + t) * a.H + h]);
            gcs[t] = run;
        }
    }
    __syncthreads();
    const float glast = gcs[n - 1];
    for (int t = threadIdx.x; t < n; t += 256) {
        gv[t] = gcs[t];
        gv[DN_C + t] = qk_expf(gcs[t]);
        gv[2 * DN_C + t] = qk_expf(__fsub_rn(glast, gcs[t]));
    }
    if (threadIdx.x == 0) gv[3 * DN_C] = qk_expf(glast);
    float *dm = s.dm + (int64_t)h * DN_C * DN_C;
    for (int p = threadIdx.x; p < n * n; p += 256) {
        const int i = p / n, j = p % n;
        dm[i * DN_C + j] = i > j ? qk_expf(__fsub_rn(gcs[i], gcs[j])) : 0.0f;
    }
    const int64_t ho = (int64_t)h * DN_C;
    for (int p = threadIdx.x; p < n * kd; p += 256) {
        const int t = p / kd, d = p % kd;
        const float b = a.beta[(a.c0 + t) * a.H + h];
        const float kbv = __fmul_rn(row_of(a.k, a, t, h, kd)[d], b);
        const float ge = qk_expf(gcs[t]);
        s.kb[(ho + t) * kd + d] = kbv;
        s.kbg[(ho + t) * kd + d] = __fmul_rn(kbv, ge);
        s.qg[(ho + t) * kd + d] = __fmul_rn(ge, row_of(a.q, a, t, h, kd)[d]);
    }
    for (int p = threadIdx.x; p < n * vd; p += 256) {
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
    __shared__ float kj[16][DN_D], kbi[16][DN_D], qi[16][DN_D];
    const int64_t ho = (int64_t)h * DN_C;
    for (int p = threadIdx.x; p < 16 * kd; p += 256) {
        const int r = p / kd, d = p % kd;
        kj[r][d] = j0 + r < n ? row_of(a.k, a, j0 + r, h, kd)[d] : 0.0f;
        kbi[r][d] = i0 + r < n ? s.kb[(ho + i0 + r) * kd + d] : 0.0f;
        qi[r][d] = i0 + r < n ? row_of(a.q, a, i0 + r, h, kd)[d] : 0.0f;
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

// 3. one workgroup of 64 lanes per head, lane j solves column j:
// X[i][j] = (B[i][j] - sum_{t<i} A[i][t] X[t][j]) / A[i][i] with A = I +
// strict-lower kkd, B = -kkd (slm/chunked.c:196-213), then attn = X below
// the diagonal, 1 on it, 0 above.
__global__ __launch_bounds__(64) void k_dn_solve(DnArgs a, DnScratch s) {
    const int h = blockIdx.x, n = a.n, j = threadIdx.x;
    __shared__ float A[DN_C][DN_C + 1];
    __shared__ float X[DN_C][DN_C + 1];
    const int64_t ho = (int64_t)h * DN_C;
    for (int p = threadIdx.x; p < n * n; p += 64) {
        const int i = p / n, t = p % n;
        A[i][t] = s.kkd[(ho + i) * DN_C + t];
    }
    __syncthreads();
    if (j < n) {
        for (int i = 0; i < n; i++) {
            float acc = 0.0f;
            for (int t = 0; t < i; t++) acc = __fadd_rn(acc, __fmul_rn(A[i][t], X[t][j]));
            const float b = -A[i][j];                  // the negated kkd (zero on and above the diagonal: -0)
            X[i][j] = __fdiv_rn(__fsub_rn(b, acc), 1.0f);   // lhs has a unit diagonal
        }
        for (int i = 0; i < n; i++)
            s.attn[(ho + i) * DN_C + j] = j < i ? X[i][j] : (j == i ? 1.0f : 0.0f);
    }
}

// 4. grid (n*max(kd,vd)/256 workgroups, H): lane (i, e)
__global__ __launch_bounds__(256) void k_dn_apply(DnArgs a, DnScratch s) {
    const int h = blockIdx.y, n = a.n, kd = a.kd, vd = a.vd;
    const int w = kd > vd ? kd : vd;
    const int p = blockIdx.x * 256 + threadIdx.x;
    if (p >= n * w) return;
    const int i = p / w, e = p % w;
    const int64_t ho = (int64_t)h * DN_C;
    const float *arow = s.attn + (ho + i) * DN_C;
    if (e < vd) {
        float acc = 0.0f;
        for (int j = 0; j <= i; j++) {
            const float c = arow[j];
            if (c == 0.0f) continue;
            acc = __fadd_rn(acc, __fmul_rn(c, s.vb[(ho + j) * vd + e]));
        }
        s.veff[(ho + i) * vd + e] = acc;
    }
    if (e < kd) {
        float acc = 0.0f;
        for (int j = 0; j <= i; j++) {
            const float c = arow[j];
            if (c == 0.0f) continue;
            acc = __fadd_rn(acc, __fmul_rn(c, s.kbg[(ho + j) * kd + e]));
        }
        s.kcd[(ho + i) * kd + e] = acc;
    }
}

// 5. grid (n*vd/256, H): lane (t, e) against the state carried in
__global__ __launch_bounds__(256) void k_dn_state_in(DnArgs a, DnScratch s) {
    const int h = blockIdx.y, n = a.n, kd = a.kd, vd = a.vd;
    const int p = blockIdx.x * 256 + threadIdx.x;
    if (p >= n * vd) return;
    const int t = p / vd, e = p % vd;
    const int64_t ho = (int64_t)h * DN_C;
    const float *st = a.state + (int64_t)h * kd * vd;
    const float *qg = s.qg + (ho + t) * kd, *kc = s.kcd + (ho + t) * kd;
    float ai = 0.0f, vp = 0.0f;
    for (int d = 0; d < kd; d++) {
        const float c = qg[d];
        if (c == 0.0f) continue;
        ai = __fadd_rn(ai, __fmul_rn(c, st[(int64_t)d * vd + e]));
    }
    for (int d = 0; d < kd; d++) {
        const float c = kc[d];
        if (c == 0.0f) continue;
        vp = __fadd_rn(vp, __fmul_rn(c, st[(int64_t)d * vd + e]));
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
    float acc = 0.0f;
    for (int u = 0; u < n; u++) acc = __fadd_rn(acc, __fmul_rn(kq[u], s.vnew[(ho + u) * vd + e]));
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
    float acc = 0.0f;
    for (int t = 0; t < n; t++) {
        const float kg = __fmul_rn(row_of(a.k, a, t, h, kd)[d], gv[2 * DN_C + t]);
        acc = __fadd_rn(acc, __fmul_rn(kg, s.vnew[(ho + t) * vd + e]));
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
    const int w = kd > vd ? kd : vd;
    for (int64_t c0 = 0; c0 < n_tok; c0 += DN_C) {
        DnArgs a{q, k, v, g, beta, state, out, c0, (int32_t)(n_tok - c0 < DN_C ? n_tok - c0 : DN_C), H, kd, vd};
        const int n = a.n;
        hipLaunchKernelGGL(k_dn_prep, dim3(H), dim3(256), 0, st, a, s);
        hipLaunchKernelGGL(k_dn_dots, dim3(4, 4, H), dim3(256), 0, st, a, s);
        hipLaunchKernelGGL(k_dn_solve, dim3(H), dim3(64), 0, st, a, s);
        hipLaunchKernelGGL(k_dn_apply, dim3((n * w + 255) / 256, H), dim3(256), 0, st, a, s);
        hipLaunchKernelGGL(k_dn_state_in, dim3((n * vd + 255) / 256, H), dim3(256), 0, st, a, s);
        hipLaunchKernelGGL(k_dn_out, dim3((n * vd + 255) / 256, H), dim3(256), 0, st, a, s);
        hipLaunchKernelGGL(k_dn_state_out, dim3((kd * vd + 255) / 256, H), dim3(256), 0, st, a, s);
    }
    return hipGetLastError();
}

}  // namespace qk
