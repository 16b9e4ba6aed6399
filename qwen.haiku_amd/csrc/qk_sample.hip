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
//  * per block of logits: the block's k largest values, sorted
//    (k_smp_blocks); the k-th largest value T_b of everything before the
//    block, by bisection over the union of those lists (held in LDS);
//    then, for the block's logits above T_b, the exact count of earlier
//    logits >= them (the earlier logits above T_b, fewer than k, plus the
//    block's own earlier candidates). Those with a count below k are the
//    entering events, listed in index order with their values
//    (k_smp_events);
//  * one wave gathers the events into LDS, replays them in order on the k
//    slots, then runs the rest of the chain on the k survivors as the
//    reference writes it (k_smp_finish).
// A NaN logit after the first k never enters and never compares >=, so it
// counts as -inf; a NaN among the first k breaks the prefix argument
// (comparisons with it are false), so k_smp_finish then runs
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

__global__ __launch_bounds__(256) void k_smp_argmax_part(const float *logits, int64_t n, ArgPart *part) {
    __shared__ ArgPart sh[4];
    float bv = 0.0f;
    int32_t bi = -1;
    const int64_t base = (int64_t)blockIdx.x * SMP_BLOCK;
    for (int j = 0; j < SMP_BLOCK / 256; j++) {
        const int64_t i = base + j * 256 + threadIdx.x;
        if (i < n) {
            const float v = logits[i];
            if (v == v) arg_better(bv, bi, v, (int32_t)i);
        }
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
// k_smp_finish then runs topk_collect literally.
constexpr int SMP_LIST_MAX = 16384;                    // floats of top-k lists (64 KB of LDS)

__device__ __forceinline__ float smp_load(const float *logits, int64_t n, int64_t i, int32_t k, int32_t &nan_fill) {
    if (i >= n) return -__builtin_inff();
    const float x = logits[i];
    if (x != x) {
        if (i < k) nan_fill = 1;
        return -__builtin_inff();
    }
    return x;
}

// Per block: its k largest values (a multiset, in no particular order)
// and whether the initial fill holds a NaN. The k-th largest key T is
// found by bisection over the block's keys (held in registers); the list
// is every value above T plus copies of T up to k.
constexpr int SMP_PER_MAX = 16;                        // logits per thread (sb <= 4096)

__global__ __launch_bounds__(256) void k_smp_blocks(const float *logits, int64_t n, int32_t k, int32_t sb,
                                                    float *tops, int32_t *nan_flag) {
    __shared__ int32_t wsum[4];
    __shared__ int32_t cnt_sh;
    const int64_t base = (int64_t)blockIdx.x * sb;
    const int per = sb / 256;
    int32_t nan_fill = 0;
    uint32_t key[SMP_PER_MAX];
#pragma unroll
    for (int j = 0; j < SMP_PER_MAX; j++)
        key[j] = j < per ? fkey(smp_load(logits, n, base + threadIdx.x * per + j, k, nan_fill)) : 0u;
    if (threadIdx.x == 0) cnt_sh = 0;
    uint32_t t = 0;                                    // largest key with count(>= key) >= k
    for (int bit = 31; bit >= 0; bit--) {
        const uint32_t cand = t | (1u << bit);
        int32_t c = 0;
#pragma unroll
        for (int j = 0; j < SMP_PER_MAX; j++) c += (j < per) & (key[j] >= cand);
        c = wave_sum_i(c);
        if ((threadIdx.x & 63) == 0) wsum[threadIdx.x >> 6] = c;
        __syncthreads();
        const int32_t total = wsum[0] + wsum[1] + wsum[2] + wsum[3];
        __syncthreads();
        if (total >= k) t = cand;
    }
    float *out = tops + (int64_t)blockIdx.x * k;
#pragma unroll
    for (int j = 0; j < SMP_PER_MAX; j++)
        if (j < per && key[j] > t) out[atomicAdd(&cnt_sh, 1)] = fkey_inv(key[j]);   // LDS counter
    __syncthreads();
    for (int32_t j = cnt_sh + threadIdx.x; j < k; j += 256) out[j] = fkey_inv(t);
    const int32_t nf = wave_sum_i(nan_fill);
    if ((threadIdx.x & 63) == 0) wsum[threadIdx.x >> 6] = nf;
    __syncthreads();
    if (threadIdx.x == 0) nan_flag[blockIdx.x] = (wsum[0] | wsum[1] | wsum[2] | wsum[3]) != 0;
}

// Block b's entering events. With P = the logits before the block and
// T = the k-th largest of P (bisection over the keys of the earlier
// blocks' top-k lists, which hold every element of P that can matter),
// a logit of the block can enter only if it exceeds T; for such a logit v
// the count of earlier logits >= v is the count in R = {x in P : x > T}
// (fewer than k elements, all inside those lists) plus the count among
// the block's earlier candidates, which go in chunks of 256 with T and R
// carried forward over each chunk (so no candidate scans more than R and
// its own chunk). Events are candidates at index >= k whose count is below
// k, written in index order with their values.
__device__ __forceinline__ int32_t wg_sum(int32_t c, int32_t *wsum) {
    c = wave_sum_i(c);
    if ((threadIdx.x & 63) == 0) wsum[threadIdx.x >> 6] = c;
    __syncthreads();
    const int32_t total = wsum[0] + wsum[1] + wsum[2] + wsum[3];
    __syncthreads();
    return total;
}

// count of keys >= x among keys[0, n4 * 4), n4 uint4 groups split over
// the workgroup; four independent LDS reads in flight per step
__device__ __forceinline__ int32_t count_keys_ge(const uint4 *keys4, int32_t n4, uint32_t x) {
    int32_t c = 0;
    int32_t j = threadIdx.x;
    for (; j + 768 < n4; j += 1024) {
        const uint4 a = keys4[j], b = keys4[j + 256], d = keys4[j + 512], e = keys4[j + 768];
        c += (a.x >= x) + (a.y >= x) + (a.z >= x) + (a.w >= x) + (b.x >= x) + (b.y >= x) + (b.z >= x) +
             (b.w >= x) + (d.x >= x) + (d.y >= x) + (d.z >= x) + (d.w >= x) + (e.x >= x) + (e.y >= x) +
             (e.z >= x) + (e.w >= x);
    }
    for (; j < n4; j += 256) {
        const uint4 a = keys4[j];
        c += (a.x >= x) + (a.y >= x) + (a.z >= x) + (a.w >= x);
    }
    return c;
}

__global__ __launch_bounds__(256) void k_smp_events(const float *logits, int64_t n, int32_t k, int32_t sb,
                                                    int32_t lcap, const float *tops, int32_t *ev_idx, float *ev_val,
                                                    int32_t *ev_n) {
    extern __shared__ uint4 lds4[];
    const int32_t b = blockIdx.x;
    const int32_t nlist = b * k;                       // prefix list elements (<= lcap, lcap % 4 == 0)
    uint32_t *keys = reinterpret_cast<uint32_t *>(lds4);
    float *cv = reinterpret_cast<float *>(keys + lcap);   // sb candidate values
    int32_t *ci = reinterpret_cast<int32_t *>(cv + sb);   // sb candidate indices
    float *rp = reinterpret_cast<float *>(ci + sb);    // R: the prefix values above T (< k), then R' twice
    __shared__ int32_t wsum[4];
    __shared__ int32_t nr_sh, ncand_sh, nr2_sh;
    __shared__ uint32_t tk_sh;
    const int64_t base = (int64_t)b * sb;
    const int32_t n4 = (nlist + 3) >> 2;
    for (int32_t j0 = threadIdx.x; j0 < n4 * 4; j0 += 256 * 8) {   // eight loads in flight per round
        uint32_t kv[8];
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const int32_t j = j0 + 256 * u;
            kv[u] = j < nlist ? fkey(tops[j]) : 0u;                // 0: below all
        }
#pragma unroll
        for (int u = 0; u < 8; u++)
            if (j0 + 256 * u < n4 * 4) keys[j0 + 256 * u] = kv[u];
    }
    if (threadIdx.x == 0) nr_sh = 0;
    __syncthreads();
    uint32_t tkey = 0;
    if (b > 0) {                                       // earlier blocks are full: sb >= k
        for (int bit = 31; bit >= 0; bit--) {
            const uint32_t cand = tkey | (1u << bit);
            if (wg_sum(count_keys_ge(lds4, n4, cand), wsum) >= k) tkey = cand;
        }
        for (int32_t j = threadIdx.x; j < nlist; j += 256)
            if (keys[j] > tkey) rp[atomicAdd(&nr_sh, 1)] = fkey_inv(keys[j]);   // LDS counter; order irrelevant
    }
    // candidates in index order: thread t owns elements [t*per, t*per + per)
    const int per = sb / 256;                          // 4 .. 16
    int32_t flag = 0, nan_fill = 0;
    float x[SMP_PER_MAX];
#pragma unroll
    for (int j = 0; j < SMP_PER_MAX; j++) {
        x[j] = j < per ? smp_load(logits, n, base + threadIdx.x * per + j, k, nan_fill) : -__builtin_inff();
        const bool c = j < per && (b > 0 ? fkey(x[j]) > tkey : x[j] > -__builtin_inff());
        flag |= (int32_t)c << j;
    }
    const int32_t mycount = __builtin_popcount(flag);
    int32_t incl = mycount;                            // inclusive scan within the wave
    for (int o = 1; o < 64; o <<= 1) {
        const int32_t y = __shfl_up(incl, o);
        if ((threadIdx.x & 63) >= o) incl += y;
    }
    if ((threadIdx.x & 63) == 63) wsum[threadIdx.x >> 6] = incl;
    __syncthreads();
    int32_t off = incl - mycount;
    for (int w = 0; w < (int)(threadIdx.x >> 6); w++) off += wsum[w];
    if (threadIdx.x == 255) ncand_sh = off + mycount;
#pragma unroll
    for (int j = 0; j < SMP_PER_MAX; j++)
        if (flag >> j & 1) {
            cv[off] = x[j];                            // a candidate is never NaN
            ci[off] = (int32_t)(base + threadIdx.x * per + j);
            off++;
        }
    __syncthreads();
    const int32_t ncand = ncand_sh, nr = nr_sh;
    // The candidates in chunks of 256, in index order, with a running
    // threshold: the top k of everything before a chunk is the multiset
    // R' (the values above T', fewer than k, as keys in rk) plus k - |R'|
    // copies of T' (key 0 while fewer than k values came before). A
    // candidate at or below T' has k earlier values >= it; one above it
    // counts those in R' and its own chunk's earlier candidates. After a
    // chunk, T' becomes the k-th largest of R', the copies and the chunk
    // (a bisection), and R' the values above it.
    uint32_t *rk = reinterpret_cast<uint32_t *>(rp);  // R' (rp's values, as keys)
    uint32_t *rk2 = rk + k;                           // the next R'
    for (int32_t r = threadIdx.x; r < nr; r += 256) rk[r] = fkey(rp[r]);
    if (threadIdx.x == 0) {
        tk_sh = tkey;
        nr2_sh = nr;
    }
    __syncthreads();
    for (int32_t c0 = 0; c0 < ncand; c0 += 256) {
        const uint32_t tk = tk_sh;
        const int32_t nr2 = nr2_sh;                    // < k <= 256
        const int32_t c = c0 + threadIdx.x;
        const bool act = c < ncand;
        const uint32_t kv = act ? fkey(cv[c]) : 0u;
        if (act && ci[c] >= k && kv > tk) {            // the initial fill never enters
            int32_t cnt = 0, r = 0;
            for (; r + 8 <= nr2; r += 8) {             // eight independent reads per step
                const uint4 a = *reinterpret_cast<const uint4 *>(&rk[r]);
                const uint4 b2 = *reinterpret_cast<const uint4 *>(&rk[r + 4]);
                cnt += (a.x >= kv) + (a.y >= kv) + (a.z >= kv) + (a.w >= kv) + (b2.x >= kv) + (b2.y >= kv) +
                       (b2.z >= kv) + (b2.w >= kv);
            }
            for (; r < nr2; r++) cnt += rk[r] >= kv;
            const float v = cv[c];
            int32_t e = c0;
            for (; e + 8 <= c && cnt < k; e += 8)
                cnt += (cv[e] >= v) + (cv[e + 1] >= v) + (cv[e + 2] >= v) + (cv[e + 3] >= v) + (cv[e + 4] >= v) +
                       (cv[e + 5] >= v) + (cv[e + 6] >= v) + (cv[e + 7] >= v);
            for (; e < c && cnt < k; e++) cnt += cv[e] >= v;
            if (cnt < k) ci[c] |= (int32_t)0x80000000;   // indices are < 2^31
        }
        if (c0 + 256 >= ncand) break;                  // uniform: the last chunk
        __syncthreads();                               // every count has read rk
        if (threadIdx.x < 64) {                        // one wave: the next T' and R'
            const int lane = threadIdx.x;
            const int32_t nc = ncand - c0 < 256 ? ncand - c0 : 256;
            uint32_t key8[8];                          // R' entries l + 64m, chunk entries l + 64m
#pragma unroll
            for (int m = 0; m < 4; m++) {
                key8[m] = lane + 64 * m < nr2 ? rk[lane + 64 * m] : 0u;
                key8[4 + m] = lane + 64 * m < nc ? fkey(cv[c0 + lane + 64 * m]) : 0u;
            }
            // bisection; each step's count is eight ballots' popcounts, so
            // the step is a short scalar chain (0 keys are padding:
            // cand >= 1)
            uint32_t t = 0;
            for (int bit = 31; bit >= 0; bit--) {
                const uint32_t cand = t | (1u << bit);
                int32_t cnt = tk >= cand ? k - nr2 : 0;
#pragma unroll
                for (int m = 0; m < 8; m++) cnt += __builtin_popcountll(__ballot(key8[m] >= cand));
                if (cnt >= k) t = cand;
            }
            int32_t nn = 0;                            // R'' = the keys above t, compacted by the wave
#pragma unroll
            for (int m = 0; m < 8; m++) {
                const bool keep = key8[m] > t;
                const uint64_t bal = __ballot(keep);
                if (keep) rk2[nn + __builtin_popcountll(bal & ((1ull << lane) - 1))] = key8[m];
                nn += __builtin_popcountll(bal);
            }
            for (int32_t r = lane; r < nn; r += 64) rk[r] = rk2[r];   // nn < k; the wave wrote rk2 itself
            if (lane == 0) {
                tk_sh = t;
                nr2_sh = nn;
            }
        }
        __syncthreads();
    }
    __syncthreads();
    if (threadIdx.x < 64) {                            // compact the events in order
        int32_t written = 0;
        for (int32_t c0 = 0; c0 < ncand; c0 += 64) {
            const int32_t c = c0 + threadIdx.x;
            const bool is_ev = c < ncand && ci[c] < 0;
            const uint64_t m = __ballot(is_ev);
            if (is_ev) {
                const int32_t pos = written + __builtin_popcountll(m & ((1ull << threadIdx.x) - 1));
                ev_idx[base + pos] = ci[c] & 0x7fffffff;
                ev_val[base + pos] = cv[c];
            }
            written += __builtin_popcountll(m);
        }
        if (threadIdx.x == 0) ev_n[b] = written;
    }
}

// ---- the final slots without a replay -------------------------------------------
// When the k fill values and the entering events are all distinct, the
// replay has a closed form. Each event evicts the smallest slot value,
// and what enters is larger than what leaves, so the evicted values come
// out strictly increasing: the j-th event (in index order) evicts the
// element of rank j among all N = k + events elements (the N - k
// smallest are exactly the evicted ones, the k largest the survivors).
// That element sits in its own fill slot, or in the slot of the earlier
// event that brought it in, so every event's slot is found by pointer
// jumping over "evicts the element of rank j". One workgroup sorts the
// elements by key (a bitonic sort in LDS), resolves the chains and writes
// each survivor into its slot; k_smp_finish then skips its replay. Ties
// (equal keys, -0 and +0 included), a NaN in the fill or more than
// SMP_NMAX elements leave *ok = 0 and the replay runs.
constexpr int SMP_NMAX = 4096;
constexpr int SMP_NSORT = 4096;                        // sort capacity: a power of two >= SMP_NMAX

__global__ __launch_bounds__(1024) void k_smp_slots(const float *logits, int64_t n, int32_t k, int32_t sb,
                                                    int32_t nblk, const int32_t *ev_idx, const float *ev_val,
                                                    const int32_t *ev_n, const int32_t *nan_flag, float *res_val,
                                                    int32_t *res_idx, int32_t *ok) {
    // (key << 32 | element) pairs, sorted ascending; then, as 32-bit
    // words, the element of each rank and the resolved slots
    __shared__ uint64_t buf[SMP_NSORT];
    __shared__ int32_t off[SMP_KMAX + 1];
    __shared__ int32_t skip;
    int32_t *byr = reinterpret_cast<int32_t *>(buf);
    const int tid = threadIdx.x;
    if (tid < 64) {
        // event offsets: wave-parallel exclusive scan, lane l owning blocks
        // 4l .. 4l+3 (every load in flight at once); NaN in the fill
        const int lane = tid;
        int32_t nf = 0, c4[4], own = 0;
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const int32_t b = 4 * lane + q;
            nf |= b < nblk ? nan_flag[b] : 0;
            c4[q] = b < nblk ? ev_n[b] : 0;
            own += c4[q];
        }
        const bool nan_fill = __ballot(nf != 0) != 0;
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
        const int32_t total = __builtin_amdgcn_readlane(incl, 63);
        if (lane == 0) {
            off[nblk] = total;
            skip = nan_fill || n <= k || total == 0 || k + total > SMP_NMAX;
            if (skip) *ok = 0;
        }
    }
    __syncthreads();
    if (skip) return;                                  // uniform
    const int32_t total = off[nblk], N = k + total;
    // element e: the fill slot e < k, or event e - k (in index order)
    auto locate = [&](int32_t j) -> int64_t {          // scratch position of event j
        int32_t lo = 0, hi = nblk;                     // last block with off[block] <= j
        while (hi - lo > 1) {
            const int32_t mid = (lo + hi) >> 1;
            if (off[mid] <= j) lo = mid;
            else hi = mid;
        }
        return (int64_t)lo * sb + (j - off[lo]);
    };
    int32_t P = 2;
    while (P < N) P <<= 1;                             // <= SMP_NSORT
    for (int32_t e = tid; e < P; e += 1024) {
        uint64_t v = ~0ull;                            // padding sorts last
        if (e < N) {
            const float x = e < k ? logits[e] : ev_val[locate(e - k)];
            v = ((uint64_t)fkey(x) << 32) | (uint32_t)e;
        }
        buf[e] = v;
    }
    __syncthreads();
    for (int32_t size = 2; size <= P; size <<= 1) {    // bitonic sort, ascending
        for (int32_t stride = size >> 1; stride > 0; stride >>= 1) {
            for (int32_t i = tid; i < (P >> 1); i += 1024) {
                const int32_t lo = 2 * i - (i & (stride - 1)), hi = lo + stride;
                const uint64_t a = buf[lo], b = buf[hi];
                const bool up = (lo & size) == 0;
                if ((a > b) == up) {
                    buf[lo] = b;
                    buf[hi] = a;
                }
            }
            __syncthreads();
        }
    }
    // ties (equal keys, -0 and +0 included) leave the order to the replay
    int tie = 0;
    for (int32_t r = 1 + tid; r < N; r += 1024) tie |= (buf[r] >> 32) == (buf[r - 1] >> 32);
    if (__syncthreads_or(tie)) {
        if (tid == 0) *ok = 0;
        return;
    }
    // ranks -> elements, in place: every thread reads its entries first
    int32_t mine[SMP_NSORT / 1024];
#pragma unroll
    for (int q = 0; q < SMP_NSORT / 1024; q++) {
        const int32_t r = tid + 1024 * q;
        mine[q] = r < N ? (int32_t)(uint32_t)buf[r] : 0;
    }
    __syncthreads();
#pragma unroll
    for (int q = 0; q < SMP_NSORT / 1024; q++) {
        const int32_t r = tid + 1024 * q;
        if (r < N) byr[r] = mine[q];
    }
    __syncthreads();
    // event j evicts element byr[j]: a fill slot, or event byr[j] - k's slot
    for (int32_t len = 1; len < 2 * total; len <<= 1) {
        for (int32_t j = tid; j < total; j += 1024) {
            const int32_t p = byr[j];
            if (p >= k) byr[j] = byr[p - k];
        }
        __syncthreads();
    }
    for (int32_t r = total + tid; r < N; r += 1024) {    // the survivors into their slots
        const int32_t e = byr[r];
        const int32_t slot = e < k ? e : byr[e - k];
        if (e < k) {
            res_val[slot] = logits[e];
            res_idx[slot] = e;
        } else {
            const int64_t at = locate(e - k);
            res_val[slot] = ev_val[at];
            res_idx[slot] = ev_idx[at];
        }
    }
    if (tid == 0) *ok = 1;
}

// One wave: the k slots (LDS), the replay of the events, then the rest of
// sample_with on lane 0.
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

__device__ __forceinline__ void smp_finish(const float *logits, int64_t n, SmpArgs a, const int32_t *ev_idx,
                                           const float *ev_val, const int32_t *ev_n, const int32_t *nan_flag,
                                           const float *res_val, const int32_t *res_idx, const int32_t *res_ok,
                                           uint64_t *rng, int32_t *token) {
    __shared__ float val[SMP_KMAX];
    __shared__ int32_t idx[SMP_KMAX];
    __shared__ int32_t off[SMP_KMAX + 1];              // event offsets per block (nblk <= 256)
    __shared__ float sp[SMP_KMAX];                     // probabilities in sorted order
    __shared__ int32_t si[SMP_KMAX];
    const int lane = threadIdx.x;
    const int32_t k = a.k, nblk = a.nblk;
    const int32_t filled = (int32_t)(n < k ? n : k);
    // NaN in the fill; event offsets (wave-parallel exclusive scan, lane l
    // owning blocks 4l .. 4l+3)
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
    const int32_t total = __builtin_amdgcn_readlane(incl, 63);
    if (lane == 0) off[nblk] = total;
    float sv[SMP_Q];
    int32_t sx[SMP_Q];
    const bool resolved = *res_ok != 0;                // k_smp_slots placed the survivors
#pragma unroll
    for (int q = 0; q < SMP_Q; q++) {
        const int32_t s_ = q * 64 + lane;
        sv[q] = s_ < filled ? (resolved ? res_val[s_] : logits[s_]) : 0.0f;
        sx[q] = resolved && s_ < filled ? res_idx[s_] : s_;
    }
    __syncthreads();
    if (!resolved && !nan_in_fill && n > k && total > 0) {
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
                if (!(v > mv)) continue;               // not reached when the events are exact
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
    }
#pragma unroll
    for (int q = 0; q < SMP_Q; q++) {
        const int32_t s_ = q * 64 + lane;
        if (s_ < filled) {
            val[s_] = sv[q];
            idx[s_] = sx[q];
        }
    }
    __syncthreads();
    if (nan_in_fill) {
        if (lane == 0) {
            if (n > k)                                 // topk_collect as written (slm/sampler.c:74-92)
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
        return;
    }
    // topk_softmax (slm/sampler.c:97-111): the max (its value is all that
    // matters), the exponentials, their sum in slot order, the division
    uint32_t mk = 0;
#pragma unroll
    for (int q = 0; q < SMP_Q; q++)
        if (q * 64 + lane < filled) mk = max(mk, fkey(sv[q]));
    mk = ~wave_min_u(~mk);
    const float m = fkey_inv(mk);
    float pe[SMP_Q];
    int32_t bad = 0;
#pragma unroll
    for (int q = 0; q < SMP_Q; q++) {
        pe[q] = q * 64 + lane < filled ? qk_expf(__fdiv_rn(__fsub_rn(sv[q], m), a.temperature)) : 0.0f;
        bad |= pe[q] != pe[q];
    }
    if (__ballot(bad != 0)) {                          // NaN probabilities: the literal order matters
        if (lane == 0) chain_literal(val, idx, filled, a, rng, token);
        return;
    }
    float sum = 0.0f;
#pragma unroll
    for (int q = 0; q < SMP_Q; q++)
        for (int32_t l = 0; l < 64 && q * 64 + l < filled; l++) sum = __fadd_rn(sum, readlane_f(pe[q], l));
    if (sum > 0.0f)
#pragma unroll
        for (int q = 0; q < SMP_Q; q++) pe[q] = __fdiv_rn(pe[q], sum);
    // topk_sort_desc (slm/sampler.c:116-129) is a stable sort by
    // descending value: rank = #greater + #equal in earlier slots
#pragma unroll
    for (int q = 0; q < SMP_Q; q++)
        if (q * 64 + lane < filled) val[q * 64 + lane] = pe[q];
    __syncthreads();
#pragma unroll
    for (int q = 0; q < SMP_Q; q++) {
        const int32_t s_ = q * 64 + lane;
        if (s_ < filled) {
            const float v = pe[q];
            int32_t r = 0;
            for (int32_t t = 0; t < filled; t++) {
                const float w = val[t];
                r += (w > v) | ((w == v) & (t < s_));
            }
            sp[r] = v;
            si[r] = sx[q];
        }
    }
    __syncthreads();
    float sq[SMP_Q];
#pragma unroll
    for (int q = 0; q < SMP_Q; q++) sq[q] = q * 64 + lane < filled ? sp[q * 64 + lane] : 0.0f;
    // top-p, min-p, renormalized roulette pick (slm/sampler.c:150-178); the
    // sorted probability j is register j / 64 of lane j % 64
    int32_t cutoff = filled;
    if (a.top_p > 0.0f && a.top_p < 1.0f) {
        float acc = 0.0f;
        bool done = false;
#pragma unroll
        for (int q = 0; q < SMP_Q; q++)
            for (int32_t l = 0; l < 64 && !done && q * 64 + l < filled; l++) {
                acc = __fadd_rn(acc, readlane_f(sq[q], l));
                if (acc >= a.top_p) {
                    cutoff = q * 64 + l + 1;
                    done = true;
                }
            }
    }
    if (a.min_p > 0.0f) {
        const float thresh = __fmul_rn(a.min_p, readlane_f(sq[0], 0));
        int32_t j = 1;
        bool done = false;
#pragma unroll
        for (int q = 0; q < SMP_Q; q++)
            for (int32_t l = q == 0 ? 1 : 0; l < 64 && !done; l++) {
                if (j < cutoff && readlane_f(sq[q], l) >= thresh) j++;
                else done = true;
            }
        cutoff = j;
    }
    float tot = 0.0f;
#pragma unroll
    for (int q = 0; q < SMP_Q; q++)
        for (int32_t l = 0; l < 64 && q * 64 + l < cutoff; l++) tot = __fadd_rn(tot, readlane_f(sq[q], l));
    uint64_t st[2] = {rng[0], rng[1]};
    const float u = __fmul_rn(rng_uniform_dev(st), tot);
    float c = 0.0f;
    int32_t picked = 0;
    bool done = false;
#pragma unroll
    for (int q = 0; q < SMP_Q; q++)
        for (int32_t l = 0; l < 64 && !done && q * 64 + l < cutoff; l++) {
            c = __fadd_rn(c, readlane_f(sq[q], l));
            if (u <= c) {
                picked = q * 64 + l;
                done = true;
            }
        }
    if (lane == 0) {
        rng[0] = st[0];
        rng[1] = st[1];
        *token = si[picked];
    }
}

// The pick, then lane 0 (which wrote the token on every path) puts the
// masked ids back.
__global__ __launch_bounds__(64) void k_smp_finish(float *logits, int64_t n, SmpArgs a, const int32_t *ev_idx,
                                                   const float *ev_val, const int32_t *ev_n, const int32_t *nan_flag,
                                                   const float *res_val, const int32_t *res_idx,
                                                   const int32_t *res_ok, uint64_t *rng, int32_t *token, SmpMask mk,
                                                   const float *saved) {
    smp_finish(logits, n, a, ev_idx, ev_val, ev_n, nan_flag, res_val, res_idx, res_ok, rng, token);
    if (threadIdx.x == 0) restore_masks(logits, n, mk, saved);
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
           + (size_t)SMP_KMAX * 8 + 16;                // resolved slots, their flag, the masked values
}

hipError_t launch_sample(float *logits, int64_t n, float temperature, int32_t k, float top_p, float min_p,
                         float penalty, int32_t window, uint64_t *rng, const int32_t *history, int32_t hist_n,
                         const int32_t *mask, int32_t n_mask, int32_t *token, void *scratch, hipStream_t s) {
    const int32_t sb = sample_block(n, k);
    const int32_t nblk = (int32_t)((n + sb - 1) / sb);
    // checked before the first launch, so a refused call leaves the logits
    // untouched (the caller's n limit keeps both)
    if (nblk > SMP_KMAX || sb > 4096 || n_mask < 0 || n_mask > 2) return hipErrorInvalidValue;
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
    float *res_val = reinterpret_cast<float *>(pr);
    int32_t *res_idx = reinterpret_cast<int32_t *>(pr + (size_t)SMP_KMAX * 4);
    int32_t *res_ok = reinterpret_cast<int32_t *>(pr + (size_t)SMP_KMAX * 8);
    float *saved = reinterpret_cast<float *>(pr + (size_t)SMP_KMAX * 8 + 8);
    const SmpMask mk{n_mask > 0 ? mask[0] : -1, n_mask > 1 ? mask[1] : -1, n_mask};

    const int32_t start = (window > 0 && window < hist_n) ? hist_n - window : 0;
    hipLaunchKernelGGL(k_smp_penalty, dim3(1), dim3(256), 0, s, logits, n, history, start, hist_n, penalty, mk.m0,
                       mk.m1, n_mask, saved);
    const int32_t w = hist_n - start;
    if (w > SMP_HIST_LDS && penalty != 1.0f)
        hipLaunchKernelGGL(k_smp_penalty_wide, dim3((unsigned)((w + 255) / 256)), dim3(256), 0, s, logits, n,
                           history + start, w, penalty);
    if (temperature <= 0.0f) {
        const int32_t ablk = (int32_t)((n + SMP_BLOCK - 1) / SMP_BLOCK);
        hipLaunchKernelGGL(k_smp_argmax_part, dim3(ablk), dim3(256), 0, s, logits, n, part);
        hipLaunchKernelGGL(k_smp_argmax_final, dim3(1), dim3(256), 0, s, logits, n, part, ablk, token, mk, saved);
        return hipGetLastError();
    }
    hipLaunchKernelGGL(k_smp_blocks, dim3(nblk), dim3(256), (size_t)sb * 4, s, logits, n, k, sb, tops, nan_flag);
    const int32_t lcap = ((nblk - 1) * k + 3) & ~3;   // the last block's prefix lists
    const size_t ev_lds = (size_t)lcap * 4 + (size_t)sb * 8 + (size_t)k * 8;
    hipLaunchKernelGGL(k_smp_events, dim3(nblk), dim3(256), ev_lds, s, logits, n, k, sb, lcap, tops, ev_idx,
                       ev_val, ev_n);
    hipLaunchKernelGGL(k_smp_slots, dim3(1), dim3(1024), 0, s, logits, n, k, sb, nblk, ev_idx, ev_val, ev_n,
                       nan_flag, res_val, res_idx, res_ok);
    SmpArgs a{temperature, top_p, min_p, k, sb, nblk};
    hipLaunchKernelGGL(k_smp_finish, dim3(1), dim3(64), 0, s, logits, n, a, ev_idx, ev_val, ev_n, nan_flag, res_val,
                       res_idx, res_ok, rng, token, mk, saved);
    return hipGetLastError();
}

}  // namespace qk
