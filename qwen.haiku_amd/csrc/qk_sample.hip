// qk_sample.hip -- the sampler chain on the device (gfx950): repetition
// penalty, greedy argmax, or topk_collect -> softmax -> sort -> top-p ->
// min-p -> roulette pick with the reference's rng, bit for bit.
//
// The reference (slm/sampler.c:134-181) scans the vocabulary once with
// topk_collect (:70-93): k slots filled with the first k logits, then each
// later logit that is strictly greater than the smallest slot value
// replaces the first slot holding that value. The softmax sums the
// survivors in slot order, so the device must end with the same slots in
// the same order, not just the same set. It does so without scanning the
// vocabulary serially:
//
//  * after any prefix the slots hold the k largest values of the prefix
//    (ties kept by the earlier element), so logit i (i >= k) enters iff
//    fewer than k earlier logits are >= it;
//  * per block of logits: the block's k largest values (k_smp_blocks);
//    the k-th largest value T_b of everything before the block, by
//    bisection over the union of those lists (held in registers, counted
//    by ballots); then, for the block's logits above T_b, the exact count
//    of earlier logits >= them (the earlier logits above T_b, fewer than
//    k, plus the block's own earlier candidates). Those with a count
//    below k are the entering events, listed in index order with their
//    values (k_smp_events);
//  * the final slots: in closed form when the values are distinct, else
//    one wave replays the events in order on the k slots; then the rest
//    of the chain on the k survivors as the reference writes it
//    (k_smp_pick).
// A NaN logit after the first k never enters and never compares >=, so it
// counts as -inf; a NaN among the first k breaks the prefix argument
// (comparisons with it are false), so k_smp_pick then runs
// topk_collect literally.
#include "qk_dev.h"
#include "qk_expf.h"
#include "qk_kernels.h"

namespace qk {

constexpr int SMP_BLOCK = 1024;                        // logits per selection block
constexpr int SMP_KMAX = 256;

// Order-preserving integer key of a non-NaN float, with -0 and +0 one key
// as IEEE comparisons (the reference's < and >) treat them.
__device__ __forceinline__ uint32_t fkey(float f) {
    const uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) == 0) return 0x80000000u;
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float fkey_inv(uint32_t k) {
    return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

// LDS ordering between the lanes of one wave, for code that not every
// wave runs (a workgroup barrier there would pair with the other waves'
// barrier somewhere else).
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
}

// Wave-wide reductions through DPP within each 16-lane row, then the four
// row results read as uniform values (every lane gets the answer).
__device__ __forceinline__ int32_t wave_sum_i(int32_t v) {
    v += dpp_xor1(v);
    v += dpp_xor2(v);
    v += dpp_hmirror(v);
    v += __builtin_amdgcn_mov_dpp(v, 0x140, 0xF, 0xF, true);   // row_mirror
    return __builtin_amdgcn_readlane(v, 0) + __builtin_amdgcn_readlane(v, 16) +
           __builtin_amdgcn_readlane(v, 32) + __builtin_amdgcn_readlane(v, 48);
}
__device__ __forceinline__ uint32_t wave_min_u(uint32_t v) {
    v = min(v, (uint32_t)dpp_xor1((int32_t)v));
    v = min(v, (uint32_t)dpp_xor2((int32_t)v));
    v = min(v, (uint32_t)dpp_hmirror((int32_t)v));
    v = min(v, (uint32_t)__builtin_amdgcn_mov_dpp((int32_t)v, 0x140, 0xF, 0xF, true));
    const uint32_t a = __builtin_amdgcn_readlane(v, 0), b = __builtin_amdgcn_readlane(v, 16);
    const uint32_t c = __builtin_amdgcn_readlane(v, 32), d = __builtin_amdgcn_readlane(v, 48);
    return min(min(a, b), min(c, d));
}

// ---- masking and repetition penalty ------------------------------------
// slm_generate_raw's min_new masking (slm/slm.c:309-322), then
// apply_rep_penalty (slm/sampler.c:49-63): for each history entry in the
// window, in order, logits[t] = lv > 0 ? lv / penalty : lv * penalty.
// Repeats of a token compound; different tokens are independent, so the
// thread owning a token's first occurrence applies its count in turn.
constexpr int SMP_HIST_LDS = 4096;                    // window entries staged in LDS

// Window entry i of h[0..w): the owner of its token's first occurrence
// applies the token's count of repeats in turn.
__device__ __forceinline__ void penalty_entry(float *logits, int64_t n, const int32_t *h, int32_t w, int32_t i,
                                              float penalty) {
    const int32_t t = h[i];
    if (t < 0 || t >= n) return;
    bool first = true;
    for (int32_t j = 0; j < i && first; j++) first = h[j] != t;
    if (!first) return;
    int32_t reps = 1;
    for (int32_t j = i + 1; j < w; j++) reps += h[j] == t;
    float v = logits[t];
    for (int32_t r = 0; r < reps; r++) v = v > 0.0f ? __fdiv_rn(v, penalty) : __fmul_rn(v, penalty);
    logits[t] = v;
}

// One workgroup: the masks, then (windows of at most SMP_HIST_LDS ids,
// staged in LDS) the penalty.
__global__ __launch_bounds__(256) void k_smp_penalty(float *logits, int64_t n, const int32_t *history,
                                                     int32_t start, int32_t hist_n, float penalty, int32_t m0,
                                                     int32_t m1, int32_t n_mask, float *saved) {
    __shared__ int32_t hw[SMP_HIST_LDS];
    // the min_new masks in the reference's order, each value saved first
    // (a repeated id saves the -inf the first mask left)
    if (threadIdx.x == 0) {
        for (int32_t i = 0; i < n_mask; i++) {
            const int32_t t = i ? m1 : m0;
            if (t >= 0 && t < n) {
                saved[i] = logits[t];
                logits[t] = -__builtin_inff();
            }
        }
    }
    __syncthreads();
    const int32_t w = hist_n - start;
    if (w > SMP_HIST_LDS) return;                      // k_smp_penalty_wide takes it
    for (int32_t i = threadIdx.x; i < w; i += 256) hw[i] = history[start + i];
    __syncthreads();
    if (penalty == 1.0f || w == 0) return;
    for (int32_t i = threadIdx.x; i < w; i += 256) penalty_entry(logits, n, hw, w, i, penalty);
}

// Windows longer than SMP_HIST_LDS: one thread per entry over as many
// workgroups as the window needs, after k_smp_penalty has set the masks.
__global__ __launch_bounds__(256) void k_smp_penalty_wide(float *logits, int64_t n, const int32_t *history,
                                                          int32_t w, float penalty) {
    const int32_t i = blockIdx.x * 256 + threadIdx.x;
    if (i < w) penalty_entry(logits, n, history, w, i, penalty);
}

// Windows of at most 64 ids skip k_smp_penalty: the first kernel of the
// chain applies the masks and the penalty, each block to the ids in its
// own range, on its staged logits, and writes the results back.
struct SmpPen {
    const int32_t *hist;                               // the window's ids
    float *saved;                                      // the masked ids' values
    int32_t w, m0, m1, n_mask;
    float penalty;
    int32_t on;                                        // 0: k_smp_penalty ran instead
};

// Wave 0 of a block whose logits [b0, b0 + len) are staged in xs: the
// masks in order, each value saved first, then the penalty with repeats
// compounding (the first occurrence of an id applies its count).
__device__ void pen_block(float *xs, float *logits, int64_t n, int64_t b0, int32_t len, const SmpPen &pp) {
    const int lane = threadIdx.x & 63;
    if (lane == 0)
        for (int32_t i = 0; i < pp.n_mask; i++) {
            const int32_t t = i ? pp.m1 : pp.m0;
            if (t >= b0 && t < b0 + len && t < n) {
                pp.saved[i] = xs[t - b0];
                xs[t - b0] = -__builtin_inff();
                logits[t] = -__builtin_inff();
            }
        }
    wave_lds_sync();
    if (pp.penalty == 1.0f || pp.w == 0) return;
    const int32_t t = lane < pp.w ? pp.hist[lane] : -1;
    uint64_t m = __ballot(t >= b0 && t < b0 + len && t < n);
    while (m) {
        const int l = __builtin_ctzll(m);
        m &= m - 1;
        const int32_t tt = __builtin_amdgcn_readlane(t, l);
        const uint64_t same = __ballot(t == tt);
        if (__builtin_ctzll(same) != l) continue;      // not the id's first occurrence
        if (lane == 0) {
            float v = xs[tt - b0];
            for (int r = __builtin_popcountll(same); r > 0; r--)
                v = v > 0.0f ? __fdiv_rn(v, pp.penalty) : __fmul_rn(v, pp.penalty);
            xs[tt - b0] = v;
            logits[tt] = v;
        }
    }
    wave_lds_sync();
}

// ---- greedy: sample_argmax (slm/model.c:401-412) ---------------------------
// First index of the largest non-NaN logit; index 0 when logits[0] is NaN
// (no later comparison can succeed then). Per block, then over blocks.
struct ArgPart {
    float v;
    int32_t i;                                         // -1: no non-NaN logit in the block
};

__device__ __forceinline__ void arg_better(float &bv, int32_t &bi, float v, int32_t i) {
    if (i < 0) return;
    if (bi < 0 || v > bv || (v == bv && i < bi)) {
        bv = v;
        bi = i;
    }
}

__device__ __forceinline__ void arg_reduce_wg(float &bv, int32_t &bi, ArgPart *sh) {
    for (int o = 32; o >= 1; o >>= 1) {
        const float ov = __shfl_xor(bv, o);
        const int32_t oi = __shfl_xor(bi, o);
        arg_better(bv, bi, ov, oi);
    }
    if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = ArgPart{bv, bi};
    __syncthreads();
    if (threadIdx.x == 0)
        for (int w = 1; w < 4; w++) arg_better(bv, bi, sh[w].v, sh[w].i);
}

__global__ __launch_bounds__(256) void k_smp_argmax_part(float *logits, int64_t n, ArgPart *part, SmpPen pp) {
    __shared__ ArgPart sh[4];
    __shared__ float xs[SMP_BLOCK];
    float bv = 0.0f;
    int32_t bi = -1;
    const int64_t base = (int64_t)blockIdx.x * SMP_BLOCK;
    float xv[SMP_BLOCK / 256];
#pragma unroll
    for (int j = 0; j < SMP_BLOCK / 256; j++) {
        const int64_t i = base + j * 256 + threadIdx.x;
        xv[j] = i < n ? logits[i] : 0.0f;
    }
    if (pp.on) {                                       // uniform
#pragma unroll
        for (int j = 0; j < SMP_BLOCK / 256; j++) xs[j * 256 + threadIdx.x] = xv[j];
        __syncthreads();
        if (threadIdx.x < 64) pen_block(xs, logits, n, base, SMP_BLOCK, pp);
        __syncthreads();
#pragma unroll
        for (int j = 0; j < SMP_BLOCK / 256; j++) xv[j] = xs[j * 256 + threadIdx.x];
    }
#pragma unroll
    for (int j = 0; j < SMP_BLOCK / 256; j++) {
        const int64_t i = base + j * 256 + threadIdx.x;
        if (i < n && xv[j] == xv[j]) arg_better(bv, bi, xv[j], (int32_t)i);
    }
    arg_reduce_wg(bv, bi, sh);
    if (threadIdx.x == 0) part[blockIdx.x] = ArgPart{bv, bi};
}

// After the pick, the masked ids get their saved values back in mask
// order, as slm_generate_raw restores eos / eot after sample_with
// (slm/slm.c:324-333); an id masked twice ends at the second save, -inf.
struct SmpMask {
    int32_t m0, m1, n;
};

__device__ __forceinline__ void restore_masks(float *logits, int64_t n, SmpMask mk, const float *saved) {
    for (int32_t i = 0; i < mk.n; i++) {
        const int32_t t = i ? mk.m1 : mk.m0;
        if (t >= 0 && t < n) logits[t] = saved[i];
    }
}

__global__ __launch_bounds__(256) void k_smp_argmax_final(float *logits, int64_t n, const ArgPart *part, int32_t nblk,
                                                          int32_t *token, SmpMask mk, const float *saved) {
    __shared__ ArgPart sh[4];
    float bv = 0.0f;
    int32_t bi = -1;
    for (int32_t b = threadIdx.x; b < nblk; b += 256) arg_better(bv, bi, part[b].v, part[b].i);
    arg_reduce_wg(bv, bi, sh);
    if (threadIdx.x == 0) {
        const float v0 = logits[0];
        *token = (v0 != v0 || bi < 0) ? 0 : bi;
        restore_masks(logits, n, mk, saved);
    }
}

// ---- sampling path ------------------------------------------------------------
// Blocks of sb logits (a power of two >= 1024, chosen by the launcher so
// that nblk * k <= SMP_LIST_MAX). A NaN logit at an index >= k never
// enters the slots and never compares >= anything, so it is read as -inf
// here; a NaN among the first k (the initial fill) is flagged instead and
// k_smp_pick then runs topk_collect literally.
constexpr int SMP_LIST_MAX = 16384;                    // keys of the prefix lists a block holds
constexpr int SMP_WG = 1024;                           // threads of the selection kernels (16 waves)
constexpr int SMP_SBMAX = 4096;                        // largest block

__device__ __forceinline__ float smp_load(const float *logits, int64_t n, int64_t i, int32_t k, int32_t &nan_fill) {
    if (i >= n) return -__builtin_inff();
    const float x = logits[i];
    if (x != x) {
        if (i < k) nan_fill = 1;
        return -__builtin_inff();
    }
    return x;
}

// ---- wave-held sorted key lists ------------------------------------------------
// A wave holds 64R keys, element e = 64r + lane in register r; the sorts
// and merges below order them descending (key 0 is padding, below every
// real key). Cross-lane exchanges go through DPP (lane ^ 1, 2, 8),
// ds_swizzle (^ 4, 16) or ds_bpermute (^ 32, and the reversal); an
// all-VALU set (row shifts, v_permlane16/32_swap) measured slower.
__device__ __forceinline__ uint32_t lane_xor(uint32_t v, int s) {
    switch (s) {
        case 1: return (uint32_t)dpp_xor1((int32_t)v);
        case 2: return (uint32_t)dpp_xor2((int32_t)v);
        case 8: return (uint32_t)__builtin_amdgcn_mov_dpp((int32_t)v, 0x128, 0xF, 0xF, true);   // row_ror:8
        case 4: return (uint32_t)__builtin_amdgcn_ds_swizzle((int32_t)v, 0x101F);
        case 16: return (uint32_t)__builtin_amdgcn_ds_swizzle((int32_t)v, 0x401F);
        default: return (uint32_t)__shfl_xor((int32_t)v, 32);
    }
}

// Lane l <- lane 63 - l.
__device__ __forceinline__ uint32_t lane_rev(uint32_t v) {
    return (uint32_t)__shfl((int32_t)v, 63 - (int)(threadIdx.x & 63));
}

// One compare-exchange stage of a bitonic network over the wave's list:
// elements e and e ^ stride, the larger first where e & size is 0 (size
// above 64R: everywhere).
template <int R>
__device__ __forceinline__ void bitonic_stage(uint32_t (&v)[R], int size, int stride) {
    const int lane = threadIdx.x & 63;
    if (stride >= 64) {
        const int d = stride / 64;
#pragma unroll
        for (int r = 0; r < R; r++)
            if (!(r & d)) {
                const int r2 = r | d;
                const bool desc = ((64 * r) & size) == 0;
                const uint32_t hi = max(v[r], v[r2]), lo = min(v[r], v[r2]);
                v[r] = desc ? hi : lo;
                v[r2] = desc ? lo : hi;
            }
    } else {
#pragma unroll
        for (int r = 0; r < R; r++) {
            const uint32_t p = lane_xor(v[r], stride);
            const bool lower = (lane & stride) == 0;
            const bool desc = ((64 * r + lane) & size) == 0;
            v[r] = lower == desc ? max(v[r], p) : min(v[r], p);
        }
    }
}

template <int R>
__device__ __forceinline__ void wave_sort_desc(uint32_t (&v)[R]) {
#pragma unroll
    for (int size = 2; size <= 64 * R; size <<= 1)
#pragma unroll
        for (int stride = size >> 1; stride > 0; stride >>= 1) bitonic_stage(v, size, stride);
}

// a := the top 64R of a and b (both sorted), sorted: max(a[e], b[64R-1-e])
// is that top as a bitonic sequence, then one bitonic merge.
template <int R>
__device__ __forceinline__ void wave_merge_top(uint32_t (&a)[R], const uint32_t (&b)[R]) {
#pragma unroll
    for (int r = 0; r < R; r++) a[r] = max(a[r], lane_rev(b[R - 1 - r]));
#pragma unroll
    for (int stride = 32 * R; stride > 0; stride >>= 1) bitonic_stage(a, 128 * R, stride);
}

// c := a and b (both sorted, 64R keys each) merged, sorted: a followed by
// b reversed is a bitonic sequence; one bitonic merge over 2R registers.
template <int R>
__device__ __forceinline__ void wave_merge_all(const uint32_t (&a)[R], const uint32_t (&b)[R], uint32_t (&c)[2 * R]) {
#pragma unroll
    for (int r = 0; r < R; r++) {
        c[r] = a[r];
        c[R + r] = lane_rev(b[R - 1 - r]);
    }
#pragma unroll
    for (int stride = 64 * R; stride > 0; stride >>= 1) bitonic_stage(c, 256 * R, stride);
}

// Every wave holds a sorted list; afterwards wave 0 holds the top 64R of
// their union, sorted (a tree of merges, four barriers). lds: 16 * 64R keys.
template <int R>
__device__ __forceinline__ void wg_merge_top(uint32_t (&v)[R], uint32_t *lds) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
    for (int l = 1; l < 16; l <<= 1) {
        if ((wave & (2 * l - 1)) == l)
#pragma unroll
            for (int r = 0; r < R; r++) lds[wave * 64 * R + 64 * r + lane] = v[r];
        __syncthreads();
        if ((wave & (2 * l - 1)) == 0) {
            uint32_t o[R];
#pragma unroll
            for (int r = 0; r < R; r++) o[r] = lds[(wave + l) * 64 * R + 64 * r + lane];
            wave_merge_top(v, o);
        }
    }
}

// List registers for k: 64R >= k.
__host__ __device__ constexpr int smp_regs(int32_t k) { return k <= 64 ? 1 : (k <= 128 ? 2 : 4); }

// Per block: its k largest values, sorted descending, and whether the
// initial fill holds a NaN. Each wave sorts its 64 * PER keys in
// registers, then a tree of merges leaves the block's top 64R in wave 0.
template <int PER, int R>
__global__ __launch_bounds__(SMP_WG) void k_smp_blocks(float *logits, int64_t n, int32_t k, float *tops,
                                                       int32_t *nan_flag, SmpPen pp) {
    __shared__ uint32_t lds[16 * 64 * R];
    __shared__ float xs[PER * SMP_WG];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t b0 = (int64_t)blockIdx.x * (PER * SMP_WG);
    const int64_t base = b0 + wave * 64 * PER;
    float xv[PER];
#pragma unroll
    for (int r = 0; r < PER; r++) {
        const int64_t i = base + 64 * r + lane;
        xv[r] = i < n ? logits[i] : 0.0f;
    }
    if (pp.on) {                                       // uniform
#pragma unroll
        for (int r = 0; r < PER; r++) xs[wave * 64 * PER + 64 * r + lane] = xv[r];
        __syncthreads();
        if (wave == 0) pen_block(xs, logits, n, b0, PER * SMP_WG, pp);
        __syncthreads();
#pragma unroll
        for (int r = 0; r < PER; r++) xv[r] = xs[wave * 64 * PER + 64 * r + lane];
    }
    int32_t nan_fill = 0;
    uint32_t v[R];
#pragma unroll
    for (int r = 0; r < R; r++) {
        v[r] = 0u;
        if (r < PER) {
            const int64_t i = base + 64 * r + lane;
            float x = i < n ? xv[r] : -__builtin_inff();
            if (x != x) {                              // as smp_load
                if (i < k) nan_fill = 1;
                x = -__builtin_inff();
            }
            v[r] = fkey(x);
        }
    }
    wave_sort_desc(v);
    const int nf = __syncthreads_or(nan_fill);
    wg_merge_top(v, lds);
    if (wave == 0) {
        float *out = tops + (int64_t)blockIdx.x * k;
#pragma unroll
        for (int r = 0; r < R; r++)
            if (64 * r + lane < k) out[64 * r + lane] = fkey_inv(v[r]);
        if (lane == 0) nan_flag[blockIdx.x] = nf;
    }
}

// Block b's entering events. With P = the logits before the block and
// T = the k-th largest of P, a logit of the block can enter only if it
// exceeds T (in block 0, anything above -inf); such a logit v enters iff
// fewer than k earlier logits are >= v. Earlier logits of the block that
// are at or below T can never be >= v, so only the top k of P and the
// block's own candidates count. Events (index >= k) are written in index
// order with their values.
//
// The top k of P is the top of the earlier blocks' sorted lists: wave w
// merges lists w, w + 16, ... (batches as trees), then a tree of merges
// across the waves. Inside the block, sub-chunk c (64 consecutive logits,
// register j of wave w for c = PER w + j) is sorted in registers; the top
// 64R of P and of the sub-chunks before c comes from a prefix scan of the
// waves' tops (Hillis-Steele over 16 waves) and the wave's own earlier
// sub-chunks. A candidate's count is then a binary search in that sorted
// top plus the earlier lanes of its sub-chunk, read lane by lane. A block
// with at most 64 candidates skips the scan: one wave holds them all.
template <int R>
__device__ __forceinline__ void wave_put(uint32_t *dst, const uint32_t (&v)[R]) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int r = 0; r < R; r++) dst[64 * r + lane] = v[r];
}
template <int R>
__device__ __forceinline__ void wave_get(uint32_t (&v)[R], const uint32_t *src) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int r = 0; r < R; r++) v[r] = src[64 * r + lane];
}

template <int PER, int R>
__global__ __launch_bounds__(SMP_WG) void k_smp_events(const float *logits, int64_t n, int32_t k,
                                                       const float *tops, int32_t *ev_idx, float *ev_val,
                                                       int32_t *ev_n) {
    constexpr int SB = PER * SMP_WG;
    constexpr int LB = 16 / R;                         // lists loaded per batch (a power of two)
    __shared__ uint32_t lds[16 * 64 * R];              // merge exchanges, then each wave's running top
    __shared__ uint32_t pb[64 * R];                    // the top of P, sorted
    __shared__ int32_t ecnt[16 * PER];                 // candidates, then events per sub-chunk; offsets
    __shared__ uint32_t c1k[64];                       // at most 64 candidates: keys, indices, values
    __shared__ int32_t c1i[64];
    __shared__ float c1v[64];
    __shared__ int32_t ncand_sh;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int32_t b = blockIdx.x;
    const int64_t base = (int64_t)b * SB;
    // the block's logits first, so their loads overlap the merges
    int32_t nan_fill = 0;
    float x[PER];
#pragma unroll
    for (int j = 0; j < PER; j++) x[j] = smp_load(logits, n, base + 64 * (wave * PER + j) + lane, k, nan_fill);
    uint32_t tkey = 0;                                 // block 0: no prefix
    if (b > 0) {                                       // earlier blocks are full: SB >= k
        uint32_t acc[R];
#pragma unroll
        for (int r = 0; r < R; r++) acc[r] = 0u;
        for (int32_t s0 = wave; s0 < b; s0 += 16 * LB) {
            uint32_t l[LB][R];
#pragma unroll
            for (int q = 0; q < LB; q++)
#pragma unroll
                for (int r = 0; r < R; r++) {
                    const int32_t sl = s0 + 16 * q, e = 64 * r + lane;
                    l[q][r] = sl < b && e < k ? fkey(tops[(int64_t)sl * k + e]) : 0u;
                }
#pragma unroll
            for (int h = 1; h < LB; h <<= 1)           // independent merges at each level
#pragma unroll
                for (int q = 0; q + h < LB; q += 2 * h)
                    if (s0 + 16 * (q + h) < b) wave_merge_top(l[q], l[q + h]);
            wave_merge_top(acc, l[0]);
        }
        wg_merge_top(acc, lds);
        if (wave == 0) wave_put(pb, acc);
        __syncthreads();
        tkey = pb[k - 1];
    }
    // keys of the candidates; 0 (counts for nothing) elsewhere
    uint32_t key[PER];
#pragma unroll
    for (int j = 0; j < PER; j++) {
        const uint32_t kx = fkey(x[j]);
        key[j] = (b > 0 ? kx > tkey : x[j] > -__builtin_inff()) ? kx : 0u;
    }
    // at most 64 candidates (every block but the first, for typical
    // logits): one wave takes them in index order, one per lane
    int32_t *cc = ecnt;
#pragma unroll
    for (int j = 0; j < PER; j++) {
        const uint64_t m = __ballot(key[j] != 0u);
        if (lane == 0) cc[wave * PER + j] = __builtin_popcountll(m);
    }
    __syncthreads();
    if (wave == 0) {                                   // exclusive scan of the candidate counts
        const int32_t c = lane < 16 * PER ? cc[lane] : 0;
        int32_t inc = c;
        for (int o = 1; o < 64; o <<= 1) {
            const int32_t y = __shfl_up(inc, o);
            if (lane >= o) inc += y;
        }
        if (lane < 16 * PER) cc[lane] = inc - c;
        if (lane == 63) ncand_sh = inc;
    }
    __syncthreads();
    const int32_t ncand = ncand_sh;
    if (ncand <= 64) {                                 // uniform
#pragma unroll
        for (int j = 0; j < PER; j++) {
            const uint64_t m = __ballot(key[j] != 0u);
            if (key[j] != 0u) {
                const int32_t pos = cc[wave * PER + j] + __builtin_popcountll(m & ((1ull << lane) - 1));
                c1k[pos] = key[j];
                c1i[pos] = (int32_t)(base + 64 * (wave * PER + j) + lane);
                c1v[pos] = x[j];
            }
        }
        __syncthreads();
        if (wave != 0) return;
        const uint32_t kv = lane < ncand ? c1k[lane] : 0u;
        const int32_t idx = lane < ncand ? c1i[lane] : 0;
        bool ev = false;
        int32_t cnt = 0;
        if (kv != 0u && idx >= k) {                    // the initial fill never enters
            if (b > 0)
#pragma unroll
                for (int step = 64 * R; step > 0; step >>= 1)
                    if (cnt + step <= k && pb[cnt + step - 1] >= kv) cnt += step;
            ev = cnt < k;
        }
        if (__ballot(ev)) {                            // plus the earlier candidates
            for (int l2 = 0; l2 < 63; l2++) {
                const uint32_t o = (uint32_t)__builtin_amdgcn_readlane((int32_t)kv, l2);
                cnt += (l2 < lane) & (o >= kv);
            }
            ev = ev && cnt < k;
        }
        const uint64_t m = __ballot(ev);
        if (ev) {
            const int32_t pos = __builtin_popcountll(m & ((1ull << lane) - 1));
            ev_idx[base + pos] = idx;
            ev_val[base + pos] = c1v[lane];
        }
        if (lane == 0) ev_n[b] = __builtin_popcountll(m);
        return;
    }
    uint32_t cl[PER][R];                               // the sub-chunks, sorted
#pragma unroll
    for (int j = 0; j < PER; j++) {
        uint32_t one[1] = {key[j]};
        wave_sort_desc(one);
        cl[j][0] = one[0];
#pragma unroll
        for (int r = 1; r < R; r++) cl[j][r] = 0u;
    }
    uint32_t top[R];                                   // the wave's sub-chunks, then the prefix before them
#pragma unroll
    for (int r = 0; r < R; r++) top[r] = cl[0][r];
#pragma unroll
    for (int j = 1; j < PER; j++) wave_merge_top(top, cl[j]);
    // inclusive scan of the waves' tops (Hillis-Steele), then shift by one
    uint32_t *my = lds + wave * 64 * R;
#pragma unroll
    for (int l = 1; l < 16; l <<= 1) {
        wave_put(my, top);
        __syncthreads();
        if (wave >= l) {
            uint32_t o[R];
            wave_get(o, lds + (wave - l) * 64 * R);
            wave_merge_top(top, o);
        }
        __syncthreads();
    }
    wave_put(my, top);
    __syncthreads();
    if (wave > 0) wave_get(top, lds + (wave - 1) * 64 * R);
    else
#pragma unroll
        for (int r = 0; r < R; r++) top[r] = 0u;
    if (b > 0) {
        uint32_t p[R];
        wave_get(p, pb);
        wave_merge_top(top, p);
    }
    __syncthreads();                                   // every wave has read the scan's slots
    // (ecnt is free again: every wave read its candidate offsets before the
    // scan's barriers) counts, sub-chunk by sub-chunk; `top` is the sorted top of everything
    // before the sub-chunk
    int32_t evf = 0;
#pragma unroll
    for (int j = 0; j < PER; j++) {
        if (j > 0) wave_merge_top(top, cl[j - 1]);
        wave_put(my, top);
        wave_lds_sync();
        const uint32_t kv = key[j];
        const int64_t idx = base + 64 * (wave * PER + j) + lane;
        bool ev = false;
        int32_t cnt = 0;                               // leading entries of the top >= v
        if (kv != 0u && idx >= k) {                    // the initial fill never enters
#pragma unroll
            for (int step = 64 * R; step > 0; step >>= 1)
                if (cnt + step <= k && my[cnt + step - 1] >= kv) cnt += step;
            ev = cnt < k;
        }
        if (__ballot(ev)) {                            // plus the earlier lanes of the sub-chunk
            for (int l2 = 0; l2 < 63; l2++) {
                const uint32_t o = (uint32_t)__builtin_amdgcn_readlane((int32_t)kv, l2);
                cnt += (l2 < lane) & (o >= kv);
            }
            ev = ev && cnt < k;
        }
        wave_lds_sync();                               // the slot is rewritten for the next sub-chunk
        const uint64_t m = __ballot(ev);
        evf |= (int32_t)ev << j;
        if (lane == 0) ecnt[wave * PER + j] = __builtin_popcountll(m);
    }
    __syncthreads();
    if (wave == 0) {                                   // exclusive scan of the counts, in index order
        const int32_t c = lane < 16 * PER ? ecnt[lane] : 0;
        int32_t inc = c;
        for (int o = 1; o < 64; o <<= 1) {
            const int32_t y = __shfl_up(inc, o);
            if (lane >= o) inc += y;
        }
        if (lane < 16 * PER) ecnt[lane] = inc - c;
        if (lane == 63) ev_n[b] = inc;
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < PER; j++) {
        const bool ev = evf >> j & 1;
        const uint64_t m = __ballot(ev);
        if (ev) {
            const int32_t pos = ecnt[wave * PER + j] + __builtin_popcountll(m & ((1ull << lane) - 1));
            ev_idx[base + pos] = (int32_t)(base + 64 * (wave * PER + j) + lane);
            ev_val[base + pos] = x[j];
        }
    }
}

struct SmpArgs {
    float temperature, top_p, min_p;
    int32_t k, sb, nblk;
};

__device__ __forceinline__ uint64_t rotl64(uint64_t x, int s) { return (x << s) | (x >> (64 - s)); }

// rng_next then rng_uniform (slm/model.c:420-447)
__device__ __forceinline__ float rng_uniform_dev(uint64_t *st) {
    const uint64_t s0 = st[0];
    uint64_t s1 = st[1];
    const uint64_t out = rotl64(s0 * 5, 7) * 9;
    s1 ^= s0;
    st[0] = rotl64(s0, 24) ^ s1 ^ (s1 << 16);
    st[1] = rotl64(s1, 37);
    return __fdiv_rn((float)(uint32_t)(out >> 40), 16777216.0f);
}

// Slot s lives in register q = s / 64 of lane s % 64 while the events are
// replayed; `worst` (the first slot holding the smallest value) is found
// with a DPP minimum over the keys and a ballot per register.
constexpr int SMP_Q = SMP_KMAX / 64;

__device__ __forceinline__ void slot_min(const float (&sv)[SMP_Q], int32_t k, float &mv, int32_t &ms) {
    uint32_t lk = 0xffffffffu;
#pragma unroll
    for (int q = 0; q < SMP_Q; q++)
        if (q * 64 + (int)threadIdx.x < k) lk = min(lk, fkey(sv[q]));
    const uint32_t mk = wave_min_u(lk);
    ms = 0;
#pragma unroll
    for (int q = SMP_Q - 1; q >= 0; q--) {
        const uint64_t m = __ballot(q * 64 + (int)threadIdx.x < k && fkey(sv[q]) == mk);
        if (m) ms = q * 64 + __builtin_ctzll(m);
    }
    mv = fkey_inv(mk);
}

__device__ __forceinline__ float readlane_f(float v, int32_t l) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}

// The events of positions [e0, e0 + 64) as lane values (idx -1 past the end).
__device__ __forceinline__ void gather_events(const int32_t *off, int32_t nblk, int32_t sb, int32_t e0,
                                              int32_t total, const int32_t *ev_idx, const float *ev_val,
                                              int32_t &gi, float &gv) {
    const int32_t e = e0 + (int32_t)threadIdx.x;
    gi = -1;
    gv = 0.0f;
    if (e < total) {
        int32_t lo = 0, hi = nblk;                     // last block with off[block] <= e
        while (hi - lo > 1) {
            const int32_t mid = (lo + hi) >> 1;
            if (off[mid] <= e) lo = mid;
            else hi = mid;
        }
        const int64_t a = (int64_t)lo * sb + (e - off[lo]);
        gi = ev_idx[a];
        gv = ev_val[a];
    }
}

// The tail of sample_with exactly as written (slm/sampler.c:97-181) on
// lane 0, for slots holding NaN or probabilities that come out NaN.
__device__ void chain_literal(float *val, int32_t *idx, int32_t filled, const SmpArgs &a, uint64_t *rng,
                              int32_t *token) {
    float m = val[0];
    for (int32_t j = 1; j < filled; j++)
        if (val[j] > m) m = val[j];
    float sum = 0.0f;
    for (int32_t j = 0; j < filled; j++) {
        val[j] = qk_expf(__fdiv_rn(__fsub_rn(val[j], m), a.temperature));
        sum = __fadd_rn(sum, val[j]);
    }
    if (sum > 0.0f)
        for (int32_t j = 0; j < filled; j++) val[j] = __fdiv_rn(val[j], sum);
    for (int32_t i = 1; i < filled; i++) {
        const float v = val[i];
        const int32_t id = idx[i];
        int32_t j = i - 1;
        while (j >= 0 && val[j] < v) {
            val[j + 1] = val[j];
            idx[j + 1] = idx[j];
            j--;
        }
        val[j + 1] = v;
        idx[j + 1] = id;
    }
    int32_t cutoff = filled;
    if (a.top_p > 0.0f && a.top_p < 1.0f) {
        float acc = 0.0f;
        for (int32_t j = 0; j < filled; j++) {
            acc = __fadd_rn(acc, val[j]);
            if (acc >= a.top_p) {
                cutoff = j + 1;
                break;
            }
        }
    }
    if (a.min_p > 0.0f) {
        const float thresh = __fmul_rn(a.min_p, val[0]);
        int32_t j = 1;
        while (j < cutoff && val[j] >= thresh) j++;
        cutoff = j;
    }
    float tot = 0.0f;
    for (int32_t j = 0; j < cutoff; j++) tot = __fadd_rn(tot, val[j]);
    uint64_t st[2] = {rng[0], rng[1]};
    const float u = __fmul_rn(rng_uniform_dev(st), tot);
    rng[0] = st[0];
    rng[1] = st[1];
    float c = 0.0f;
    int32_t picked = 0;
    for (int32_t j = 0; j < cutoff; j++) {
        c = __fadd_rn(c, val[j]);
        if (u <= c) {
            picked = j;
            break;
        }
    }
    *token = idx[picked];
}

// ---- the slots and the pick ------------------------------------------------------
// When the k fill values and the entering events are all distinct, the
// replay has a closed form. Each event evicts the smallest slot value,
// and what enters is larger than what leaves, so the evicted values come
// out strictly increasing: the j-th event (in index order) evicts the
// element of rank j among all N = k + events elements (the N - k
// smallest are exactly the evicted ones, the k largest the survivors).
// That element sits in its own fill slot, or in the slot of the earlier
// event that brought it in, so every event's slot follows from the slots
// of earlier events. One workgroup ranks the elements (by counting for
// N <= 1024, else a bitonic sort in LDS), resolves the slots in event
// order (one wave, 64 at a time, pointer jumping inside each group) and
// places the survivors. Ties (equal keys, -0 and +0 included), a NaN in
// the fill or more than SMP_NMAX elements send it to the replay instead:
// one wave replays the events in order on the k slots. Then the rest of
// the chain: the softmax numerators, their sum in slot order and the
// quotients (wave 0), the ranking of the probabilities (every thread),
// the cut and the pick (wave 0), and the masked ids get their saved values
// back.
constexpr int SMP_NMAX = 4096;

// One level of wg_sort_keys: waves w with w % 2l == 0 merge wave w + l's
// list into theirs (exchanged through ex).
template <int RC>
__device__ __forceinline__ void sort_level(const uint32_t (&cur)[RC], uint32_t (&nxt)[2 * RC], int l, uint32_t *ex) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if ((wave & (2 * l - 1)) == l)
#pragma unroll
        for (int r = 0; r < RC; r++) ex[(wave >> 1) * 64 * RC + 64 * r + lane] = cur[r];
    __syncthreads();
    if ((wave & (2 * l - 1)) == 0) {
        uint32_t o[RC];
#pragma unroll
        for (int r = 0; r < RC; r++) o[r] = ex[((wave + l) >> 1) * 64 * RC + 64 * r + lane];
        wave_merge_all(cur, o, nxt);
    }
    __syncthreads();
}

// The keys of elements [0, N), N <= 1024 RW, sorted descending into out
// (key 0 pads): each wave sorts its 64 RW keys in registers, then four
// levels of merges leave them all in wave 0. ex: 8 * 64 * 8 RW keys.
template <int RW>
__device__ __forceinline__ void wg_sort_keys(const uint32_t *keys, int32_t N, uint32_t *ex, uint32_t *out) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    uint32_t v1[RW];
#pragma unroll
    for (int r = 0; r < RW; r++) {
        const int32_t e = wave * 64 * RW + 64 * r + lane;
        v1[r] = e < N ? keys[e] : 0u;
    }
    wave_sort_desc(v1);
    uint32_t v2[2 * RW], v4[4 * RW], v8[8 * RW], v16[16 * RW];
    sort_level(v1, v2, 1, ex);
    sort_level(v2, v4, 2, ex);
    sort_level(v4, v8, 4, ex);
    sort_level(v8, v16, 8, ex);
    if (wave == 0)
#pragma unroll
        for (int r = 0; r < 16 * RW; r++) out[64 * r + lane] = v16[r];
}

__global__ __launch_bounds__(SMP_WG) void k_smp_pick(float *logits, int64_t n, SmpArgs a, const int32_t *ev_idx,
                                                     const float *ev_val, const int32_t *ev_n,
                                                     const int32_t *nan_flag, uint64_t *rng, int32_t *token,
                                                     SmpMask mk, const float *saved) {
    __shared__ int32_t off[SMP_KMAX + 1];              // event offsets per block (nblk <= 256)
    __shared__ __align__(16) uint32_t skey[SMP_NMAX];  // element e: fill slot e < k, or event e - k
    __shared__ float sval[SMP_NMAX];
    __shared__ int32_t sid[SMP_NMAX];
    __shared__ int32_t byr[SMP_NMAX];                  // element of each rank; then the events' slots
    __shared__ uint64_t buf[SMP_NMAX];                 // (key << 32 | element), for the sort
    __shared__ __align__(16) float val[SMP_KMAX];      // the slots: values, then probabilities
    __shared__ int32_t idx[SMP_KMAX];
    __shared__ float sp[SMP_KMAX];                     // probabilities in sorted order
    __shared__ int32_t si[SMP_KMAX];
    __shared__ int32_t total_sh, nanf_sh, done_sh;
    const int tid = threadIdx.x, lane = tid & 63;
    const int32_t k = a.k, nblk = a.nblk;
    const int32_t filled = (int32_t)(n < k ? n : k);
    if (tid < 64) {
        // NaN in the fill; event offsets (wave-parallel exclusive scan,
        // lane l owning blocks 4l .. 4l+3)
        int32_t nf = 0, c4[4], own = 0;
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const int32_t b = 4 * lane + q;
            nf |= b < nblk ? nan_flag[b] : 0;
            c4[q] = b < nblk ? ev_n[b] : 0;
            own += c4[q];
        }
        const bool nan_in_fill = __ballot(nf != 0) != 0;
        int32_t incl = own;
        for (int o = 1; o < 64; o <<= 1) {
            const int32_t y = __shfl_up(incl, o);
            if (lane >= o) incl += y;
        }
        int32_t acc = incl - own;
#pragma unroll
        for (int q = 0; q < 4; q++) {
            if (4 * lane + q <= nblk) off[4 * lane + q] = acc;
            acc += c4[q];
        }
        if (lane == 0) {
            total_sh = __builtin_amdgcn_readlane(incl, 63);
            nanf_sh = nan_in_fill;
        }
    }
    __syncthreads();
    const int32_t total = n > k ? total_sh : 0;
    const bool nan_in_fill = nanf_sh != 0;
    const int32_t N = k + total;
    // scratch position of event j: the last block with off[block] <= j
    auto locate = [&](int32_t j) -> int64_t {
        int32_t lo = 0, hi = nblk;
        while (hi - lo > 1) {
            const int32_t mid = (lo + hi) >> 1;
            if (off[mid] <= j) lo = mid;
            else hi = mid;
        }
        return (int64_t)lo * a.sb + (j - off[lo]);
    };
    // the closed form applies: no NaN in the fill, events to place, room
    bool closed = !nan_in_fill && total > 0 && N <= SMP_NMAX;
    if (closed) {                                      // uniform
        for (int32_t e = tid; e < N; e += SMP_WG) {
            float x;
            int32_t id;
            if (e < k) {
                x = logits[e];
                id = e;
            } else {
                const int64_t at = locate(e - k);
                x = ev_val[at];
                id = ev_idx[at];
            }
            skey[e] = fkey(x);
            sval[e] = x;
            sid[e] = id;
        }
        __syncthreads();
        int tie = 0;
        if (N <= 2 * SMP_WG) {                         // sorted in registers; ranks by binary search
            uint32_t *sorted = reinterpret_cast<uint32_t *>(buf);   // 2048 keys, then the exchange area
            uint32_t *ex = sorted + 2 * SMP_WG;
            if (N <= SMP_WG) wg_sort_keys<1>(skey, N, ex, sorted);
            else wg_sort_keys<2>(skey, N, ex, sorted);
            __syncthreads();
            for (int32_t e = tid; e < N; e += SMP_WG) {
                const uint32_t kv = skey[e];
                int32_t pos = 0;                       // keys above kv
                for (int32_t step = 2 * SMP_WG; step > 0; step >>= 1)
                    if (pos + step <= N && sorted[pos + step - 1] > kv) pos += step;
                tie |= pos + 1 < N && sorted[pos + 1] == kv;   // another key equal to kv
                byr[N - 1 - pos] = e;
            }
        } else {                                       // bitonic sort of (key, element), ascending
            int32_t P = 2;
            while (P < N) P <<= 1;                     // <= SMP_NMAX
            for (int32_t e = tid; e < P; e += SMP_WG)
                buf[e] = e < N ? ((uint64_t)skey[e] << 32) | (uint32_t)e : ~0ull;   // padding sorts last
            __syncthreads();
            for (int32_t size = 2; size <= P; size <<= 1) {
                for (int32_t stride = size >> 1; stride > 0; stride >>= 1) {
                    for (int32_t i = tid; i < (P >> 1); i += SMP_WG) {
                        const int32_t lo = 2 * i - (i & (stride - 1)), hi = lo + stride;
                        const uint64_t x0 = buf[lo], x1 = buf[hi];
                        const bool up = (lo & size) == 0;
                        if ((x0 > x1) == up) {
                            buf[lo] = x1;
                            buf[hi] = x0;
                        }
                    }
                    __syncthreads();
                }
            }
            for (int32_t r = tid; r < N; r += SMP_WG) {
                byr[r] = (int32_t)(uint32_t)buf[r];
                tie |= r > 0 && (buf[r] >> 32) == (buf[r - 1] >> 32);
            }
        }
        closed = !__syncthreads_or(tie);               // ties leave the order to the replay
    }
    if (closed) {
        if (tid < 64) {                                // event j's slot, in event order
            for (int32_t c0 = 0; c0 < total; c0 += 64) {
                const int32_t j = c0 + lane;
                int32_t p = j < total ? byr[j] : 0;    // the element event j evicts
                int32_t slot = p, d = -1;              // resolved slot, or the in-group event it waits on
                if (j < total && p >= k) {
                    if (p - k < c0) slot = byr[p - k];   // an earlier group: resolved already
                    else d = p - k - c0;               // an earlier lane of this group
                }
                for (int it = 0; it < 6 && __ballot(d >= 0); it++) {   // pointer jumping inside the group
                    const int32_t ts = __shfl(slot, d < 0 ? lane : d);
                    const int32_t td = __shfl(d, d < 0 ? lane : d);
                    if (d >= 0) {
                        if (td < 0) {
                            slot = ts;
                            d = -1;
                        } else {
                            d = td;
                        }
                    }
                }
                wave_lds_sync();                       // every lane has read byr for this group
                if (j < total) byr[j] = slot;
                wave_lds_sync();
            }
        }
        __syncthreads();
        for (int32_t r = total + tid; r < N; r += SMP_WG) {   // the survivors into their slots
            const int32_t e = byr[r];
            const int32_t slot = e < k ? e : byr[e - k];
            val[slot] = sval[e];
            idx[slot] = sid[e];
        }
    } else {
        for (int32_t s_ = tid; s_ < filled; s_ += SMP_WG) {   // the fill
            val[s_] = logits[s_];
            idx[s_] = s_;
        }
    }
    __syncthreads();
    // Wave 0: returns true when it ran the chain to the end literally (a
    // NaN in the fill, or a NaN probability).
    auto slots_softmax = [&]() -> bool {
        float sv[SMP_Q];
        int32_t sx[SMP_Q];
#pragma unroll
        for (int q = 0; q < SMP_Q; q++) {
            const int32_t s_ = q * 64 + lane;
            sv[q] = s_ < filled ? val[s_] : 0.0f;
            sx[q] = s_ < filled ? idx[s_] : s_;
        }
        if (!closed && !nan_in_fill && total > 0) {   // the replay
            float mv;
            int32_t ms;
            slot_min(sv, k, mv, ms);
            int32_t gi, ni;
            float gv, nv;
            gather_events(off, nblk, a.sb, 0, total, ev_idx, ev_val, gi, gv);
            for (int32_t e0 = 0; e0 < total; e0 += 64) {
                gather_events(off, nblk, a.sb, e0 + 64, total, ev_idx, ev_val, ni, nv);   // next batch in flight
                const int32_t cnt = total - e0 < 64 ? total - e0 : 64;
                for (int32_t j = 0; j < cnt; j++) {
                    const float v = readlane_f(gv, j);
                    if (!(v > mv)) continue;           // not reached when the events are exact
                    const int32_t i = __builtin_amdgcn_readlane(gi, j);
                    const int32_t q = ms >> 6;
                    if (lane == (ms & 63)) {
#pragma unroll
                        for (int r = 0; r < SMP_Q; r++)
                            if (r == q) {
                                sv[r] = v;
                                sx[r] = i;
                            }
                    }
                    slot_min(sv, k, mv, ms);
                }
                gi = ni;
                gv = nv;
            }
#pragma unroll
            for (int q = 0; q < SMP_Q; q++) {
                const int32_t s_ = q * 64 + lane;
                if (s_ < filled) {
                    val[s_] = sv[q];
                    idx[s_] = sx[q];
                }
            }
            wave_lds_sync();
        }
        if (nan_in_fill) {
            if (lane == 0) {
                if (n > k)                             // topk_collect as written (slm/sampler.c:74-92)
                    for (int64_t i = k; i < n; i++) {
                        const float lv = logits[i];
                        int32_t worst = 0;
                        for (int32_t j = 1; j < k; j++)
                            if (val[j] < val[worst]) worst = j;
                        if (lv > val[worst]) {
                            idx[worst] = (int32_t)i;
                            val[worst] = lv;
                        }
                    }
                chain_literal(val, idx, filled, a, rng, token);
            }
            return true;
        }
        // topk_softmax (slm/sampler.c:97-111): the max (its value is all
        // that matters), the exponentials, their sum in slot order, the
        // division
        uint32_t mkey = 0;
#pragma unroll
        for (int q = 0; q < SMP_Q; q++)
            if (q * 64 + lane < filled) mkey = max(mkey, fkey(sv[q]));
        mkey = ~wave_min_u(~mkey);
        const float m = fkey_inv(mkey);
        float pe[SMP_Q];
        int32_t bad = 0;
#pragma unroll
        for (int q = 0; q < SMP_Q; q++) {
            pe[q] = q * 64 + lane < filled ? qk_expf(__fdiv_rn(__fsub_rn(sv[q], m), a.temperature)) : 0.0f;
            bad |= pe[q] != pe[q];
        }
        if (__ballot(bad != 0)) {                      // NaN probabilities: the literal order matters
            if (lane == 0) chain_literal(val, idx, filled, a, rng, token);
            return true;
        }
        float sum = 0.0f;                              // in slot order; slots past filled add +0
#pragma unroll
        for (int q = 0; q < SMP_Q; q++)
            if (q * 64 < filled)
#pragma unroll
                for (int l = 0; l < 64; l++) sum = __fadd_rn(sum, readlane_f(pe[q], l));
        if (sum > 0.0f)
#pragma unroll
            for (int q = 0; q < SMP_Q; q++) pe[q] = __fdiv_rn(pe[q], sum);
        // the probabilities for the ranking; -1 pads to a multiple of four
        // (below every probability, equal to none)
#pragma unroll
        for (int q = 0; q < SMP_Q; q++) {
            const int32_t s_ = q * 64 + lane;
            if (s_ < ((filled + 3) & ~3)) val[s_] = s_ < filled ? pe[q] : -1.0f;
        }
        return false;
    };
    if (tid < 64) {
        const bool done = slots_softmax();
        if (lane == 0) done_sh = done;
    }
    __syncthreads();
    const bool done = done_sh != 0;
    // topk_sort_desc (slm/sampler.c:116-129) is a stable sort by
    // descending value: rank = #greater + #equal in earlier slots; one
    // slot per thread, the probabilities read four at a time
    if (!done) {                                       // uniform; four threads per slot
        const int32_t sl = tid >> 2, t0 = (tid & 3) * 64;
        const int32_t nf4 = (filled + 3) & ~3, t1 = t0 + 64 < nf4 ? t0 + 64 : nf4;
        float v = 0.0f;
        int32_t r = 0;
        if (sl < filled) {
            v = val[sl];
#pragma unroll 4
            for (int32_t t = t0; t < t1; t += 4) {
                const float4 w = *reinterpret_cast<const float4 *>(&val[t]);
                r += (w.x > v) | ((w.x == v) & (t < sl));
                r += (w.y > v) | ((w.y == v) & (t + 1 < sl));
                r += (w.z > v) | ((w.z == v) & (t + 2 < sl));
                r += (w.w > v) | ((w.w == v) & (t + 3 < sl));
            }
        }
        r += dpp_xor1(r);                              // the quad's four parts
        r += dpp_xor2(r);
        if (sl < filled && (tid & 3) == 0) {
            sp[r] = v;
            si[r] = idx[sl];
        }
    }
    __syncthreads();
    if (tid >= 64) return;
    if (!done) {
        float sq[SMP_Q];
#pragma unroll
        for (int q = 0; q < SMP_Q; q++) sq[q] = q * 64 + lane < filled ? sp[q * 64 + lane] : 0.0f;
        // top-p, min-p, renormalized roulette pick (slm/sampler.c:150-178);
        // the sorted probability j is register j / 64 of lane j % 64. The
        // three running sums there (top-p's acc, the total over the cut,
        // the pick's c) are one sequence of adds from 0 in sorted order, so
        // one pass keeps every partial sum (lane j % 64 of pre[j / 64]);
        // entries past filled add +0.
        float pre[SMP_Q];
        float acc = 0.0f;
#pragma unroll
        for (int q = 0; q < SMP_Q; q++) {
            pre[q] = 0.0f;
            if (q * 64 < filled)
#pragma unroll
                for (int l = 0; l < 64; l++) {
                    acc = __fadd_rn(acc, readlane_f(sq[q], l));
                    pre[q] = lane == l ? acc : pre[q];
                }
        }
        // the first j meeting a per-lane predicate, or -1
        auto first = [&](auto pred) -> int32_t {
#pragma unroll
            for (int q = 0; q < SMP_Q; q++) {
                const uint64_t m = __ballot(q * 64 + lane < filled && pred(q));
                if (m) return q * 64 + (int32_t)__builtin_ctzll(m);
            }
            return -1;
        };
        int32_t cutoff = filled;
        if (a.top_p > 0.0f && a.top_p < 1.0f) {
            const int32_t j = first([&](int q) { return pre[q] >= a.top_p; });
            if (j >= 0) cutoff = j + 1;
        }
        if (a.min_p > 0.0f) {
            const float thresh = __fmul_rn(a.min_p, readlane_f(sq[0], 0));
            const int32_t c0 = cutoff;
            const int32_t j = first([&](int q) { return q * 64 + lane >= 1 && q * 64 + lane < c0 && !(sq[q] >= thresh); });
            cutoff = j >= 0 ? j : (c0 > 1 ? c0 : 1);
        }
        const int32_t lt = cutoff - 1;
        float tot = 0.0f;
#pragma unroll
        for (int q = 0; q < SMP_Q; q++)
            if (q == lt / 64) tot = readlane_f(pre[q], lt % 64);
        uint64_t st[2] = {rng[0], rng[1]};
        const float u = __fmul_rn(rng_uniform_dev(st), tot);
        const int32_t c1 = cutoff;
        const int32_t pj = first([&](int q) { return q * 64 + lane < c1 && u <= pre[q]; });
        const int32_t picked = pj >= 0 ? pj : 0;
        if (lane == 0) {
            rng[0] = st[0];
            rng[1] = st[1];
            *token = si[picked];
        }
    }
    if (lane == 0) restore_masks(logits, n, mk, saved);
}

// ---- launcher -------------------------------------------------------------------
// Block size: the smallest power of two >= 1024 with nblk * k within the
// LDS list budget (n <= QK_SAMPLE_MAX_N keeps it <= 4096 and nblk <= 256).
static int32_t sample_block(int64_t n, int32_t k) {
    int32_t sb = 1024;
    while (((n + sb - 1) / sb) * k > SMP_LIST_MAX) sb <<= 1;
    return sb;
}

size_t sample_scratch_bytes(int64_t n, int32_t k) {
    const int32_t sb = sample_block(n, k);
    const int64_t nblk = (n + sb - 1) / sb;
    return (size_t)nblk * sb * 8                       // event indices and values
           + (size_t)nblk * (size_t)k * 4              // per-block top-k lists
           + (size_t)nblk * 4 * 2                      // event counts, NaN flags
           + (size_t)((n + SMP_BLOCK - 1) / SMP_BLOCK) * sizeof(ArgPart) + 256    // greedy partials
           + 16;                                       // the masked values
}

hipError_t launch_sample(float *logits, int64_t n, float temperature, int32_t k, float top_p, float min_p,
                         float penalty, int32_t window, uint64_t *rng, const int32_t *history, int32_t hist_n,
                         const int32_t *mask, int32_t n_mask, int32_t *token, void *scratch, hipStream_t s) {
    const int32_t sb = sample_block(n, k);
    const int32_t nblk = (int32_t)((n + sb - 1) / sb);
    // checked before the first launch, so a refused call leaves the logits
    // untouched (the caller's n limit keeps both)
    if (nblk > SMP_KMAX || sb > SMP_SBMAX || n_mask < 0 || n_mask > 2) return hipErrorInvalidValue;
    uint8_t *p = static_cast<uint8_t *>(scratch);
    int32_t *ev_idx = reinterpret_cast<int32_t *>(p);
    p += (size_t)nblk * sb * 4;
    float *ev_val = reinterpret_cast<float *>(p);
    p += (size_t)nblk * sb * 4;
    float *tops = reinterpret_cast<float *>(p);
    p += (size_t)nblk * (size_t)k * 4;
    int32_t *ev_n = reinterpret_cast<int32_t *>(p);
    p += (size_t)nblk * 4;
    int32_t *nan_flag = reinterpret_cast<int32_t *>(p);
    p += (size_t)nblk * 4;
    ArgPart *part = reinterpret_cast<ArgPart *>((reinterpret_cast<uintptr_t>(p) + 15) & ~(uintptr_t)15);
    uint8_t *pr = reinterpret_cast<uint8_t *>(part + (n + SMP_BLOCK - 1) / SMP_BLOCK);
    float *saved = reinterpret_cast<float *>(pr);
    const SmpMask mk{n_mask > 0 ? mask[0] : -1, n_mask > 1 ? mask[1] : -1, n_mask};

    const int32_t start = (window > 0 && window < hist_n) ? hist_n - window : 0;
    const int32_t w = hist_n - start;
    const SmpPen pp{w > 0 ? history + start : nullptr, saved, w, mk.m0, mk.m1, n_mask, penalty, w <= 64};
    if (!pp.on) {
        hipLaunchKernelGGL(k_smp_penalty, dim3(1), dim3(256), 0, s, logits, n, history, start, hist_n, penalty,
                           mk.m0, mk.m1, n_mask, saved);
        if (w > SMP_HIST_LDS && penalty != 1.0f)
            hipLaunchKernelGGL(k_smp_penalty_wide, dim3((unsigned)((w + 255) / 256)), dim3(256), 0, s, logits, n,
                               history + start, w, penalty);
    }
    if (temperature <= 0.0f) {
        const int32_t ablk = (int32_t)((n + SMP_BLOCK - 1) / SMP_BLOCK);
        hipLaunchKernelGGL(k_smp_argmax_part, dim3(ablk), dim3(256), 0, s, logits, n, part, pp);
        hipLaunchKernelGGL(k_smp_argmax_final, dim3(1), dim3(256), 0, s, logits, n, part, ablk, token, mk, saved);
        return hipGetLastError();
    }
    // (sb, list registers): sb <= 1024 * R, since nblk * k <= SMP_LIST_MAX
    const int R = smp_regs(k);
    auto blocks = R == 1 ? k_smp_blocks<1, 1>
                : R == 2 ? (sb == 1024 ? k_smp_blocks<1, 2> : k_smp_blocks<2, 2>)
                         : (sb == 1024 ? k_smp_blocks<1, 4> : sb == 2048 ? k_smp_blocks<2, 4> : k_smp_blocks<4, 4>);
    auto events = R == 1 ? k_smp_events<1, 1>
                : R == 2 ? (sb == 1024 ? k_smp_events<1, 2> : k_smp_events<2, 2>)
                         : (sb == 1024 ? k_smp_events<1, 4> : sb == 2048 ? k_smp_events<2, 4> : k_smp_events<4, 4>);
    hipLaunchKernelGGL(blocks, dim3(nblk), dim3(SMP_WG), 0, s, logits, n, k, tops, nan_flag, pp);
    hipLaunchKernelGGL(events, dim3(nblk), dim3(SMP_WG), 0, s, logits, n, k, tops, ev_idx, ev_val, ev_n);
    SmpArgs sa{temperature, top_p, min_p, k, sb, nblk};
    hipLaunchKernelGGL(k_smp_pick, dim3(1), dim3(SMP_WG), 0, s, logits, n, sa, ev_idx, ev_val, ev_n, nan_flag, rng,
                       token, mk, saved);
    return hipGetLastError();
}

}  // namespace qk
