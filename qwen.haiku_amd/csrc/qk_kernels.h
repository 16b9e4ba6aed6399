// qk_kernels.h -- launchers shared between the kernel translation units
// and the C-ABI layer (qk_api.cpp). Host-side declarations only.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#define QK_GROUP_MAX_DEV 16
#define QK_TOPK_MAX_DEV 256

namespace qk {

// One GEMV of a launch (a row range of one weight matrix).
struct GemvDesc {
    int32_t type;          // 8, 12, 13, 14
    int32_t p;             // K-quants: 4-lane groups per row (4, 8, 16); Q8_0: rows per wave (4 or 1)
    int64_t n, k;
    const uint8_t *w;
    const uint8_t *xq;
    float *y;
    int32_t nb;            // blocks per row (k/256, or k/32 for Q8_0)
    int32_t rows_per_tile; // rows per tile (== tr)
    int32_t tr;            // rows per tile
    int32_t tile_cap;      // LDS bytes of one tile buffer
    int32_t ntiles;
    int32_t wg0;           // first workgroup of the launch serving this descriptor
    int32_t nwg;           // workgroups serving it (grid-stride over tiles)
    int32_t lds_act;       // bytes of the staged activation row
    int32_t xf32;          // 1: xq is the fp32 row (k floats), quantized by each workgroup
};

struct GemvArgs {
    GemvDesc d[QK_GROUP_MAX_DEV];
    int32_t count;
    int32_t lds_bytes;
    int32_t fused;         // float epilogue family: 1 = AVX2/VNNI
};

// Fill p / rows_per_tile / nb for a descriptor.
void gemv_plan(GemvDesc &d);
int64_t gemv_max_matrix_bytes();
// max_wg: workgroups per descriptor at most (the rest grid-stride).
hipError_t launch_gemv(GemvArgs &a, int max_wg, hipStream_t s);

hipError_t launch_quantize_q8k(const float *x, int64_t nblocks, uint8_t *xq, hipStream_t s);
hipError_t launch_quantize_q8_0(const float *x, int64_t nblocks, uint8_t *xq, hipStream_t s);
hipError_t launch_dequant(int type, const uint8_t *w, int64_t nblocks, float *y, hipStream_t s);

// LM head: Q6_K GEMV -> logits, then exact argmax / top-k selection.
// scratch must hold lmhead_cand_bytes(n, topk) bytes.
size_t lmhead_cand_bytes(int64_t n, int topk);
hipError_t launch_lmhead(const uint8_t *w, int64_t n, int64_t k, const uint8_t *xq, int topk,
                         float *logits, int32_t *argmax, int32_t *topk_idx, float *topk_val,
                         void *scratch, int fused, hipStream_t s);

// Decode chain links (qk_chain.hip). k_add_rmsnorm keeps a row in LDS:
// k * 4 bytes per workgroup.
hipError_t launch_add_rmsnorm(const float *h, const float *delta, const float *w, float eps, int64_t m, int64_t k,
                              float *h_out, float *x_out, uint8_t *xq, hipStream_t s);
hipError_t launch_silu(const float *src, float *dst, int64_t n, hipStream_t s);
hipError_t launch_swiglu(const float *gate, const float *up, int64_t n, float *act, uint8_t *xq, hipStream_t s);

// Sampler chain (qk_sample.hip); scratch must hold sample_scratch_bytes.
size_t sample_scratch_bytes(int64_t n, int32_t k);
hipError_t launch_sample(float *logits, int64_t n, float temperature, int32_t k, float top_p, float min_p,
                         float penalty, int32_t window, uint64_t *rng, const int32_t *history, int32_t hist_n,
                         const int32_t *mask, int32_t n_mask, int32_t *token, void *scratch, hipStream_t s);

// Chunked Gated DeltaNet (qk_deltanet.hip); scratch holds
// deltanet_scratch_bytes(H, kd, vd, n_tok); kd, vd <= 128.
size_t deltanet_scratch_bytes(int32_t H, int32_t kd, int32_t vd, int64_t n_tok);
hipError_t launch_deltanet(const float *q, const float *k, const float *v, const float *g, const float *beta,
                           int64_t n_tok, int32_t H, int32_t kd, int32_t vd, float *state, float *out,
                           void *scratch, hipStream_t s);

// Prefill GEMM (int8 MFMA); y[t*n + j].
hipError_t launch_gemm(int type, const uint8_t *w, int64_t n, int64_t k, const uint8_t *xq,
                       int64_t m, float *y, int fused, hipStream_t s);

// Prefill GEMM over weights repacked into int8 MFMA planes
// (qk_gemm_planes.hip): bytes of the planes of an n x k K-quant matrix (0
// for other types), the repacking, and the GEMM.
size_t gemm_planes_bytes(int type, int64_t n, int64_t k);
hipError_t launch_pack_planes(int type, const uint8_t *w, int64_t n, int64_t k, uint8_t *wp, hipStream_t s);
hipError_t launch_gemm_planes(int type, const uint8_t *wp, int64_t n, int64_t k, const uint8_t *xq, int64_t m,
                              float *y, int fused, hipStream_t s);

}  // namespace qk
