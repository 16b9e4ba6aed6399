// mfma_peak -- dense int8 MFMA throughput of this GPU, to set the measured
// ceiling beside the 5.0 POPS specification when reporting the prefill
// GEMM. Each wave runs four independent accumulator chains of
// v_mfma_i32_32x32x32_i8 (and, separately, v_mfma_i32_16x16x64_i8) on
// register operands; no memory traffic inside the timed loop. Prints one
// JSON line: {"mfma_i32_32x32x32_i8_tops": ..., "mfma_i32_16x16x64_i8_tops": ...}.
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>

typedef int32_t v4i __attribute__((ext_vector_type(4)));
typedef int32_t v16i __attribute__((ext_vector_type(16)));

#define ITER 4096
#define GRID 4096

__global__ __launch_bounds__(256) void k_mfma32(int seed, int *out) {
    const v4i a = {seed, seed + 1, seed + 2, seed + 3}, b = {seed ^ 5, seed ^ 7, seed ^ 9, seed ^ 11};
    v16i c0 = {0}, c1 = {0}, c2 = {0}, c3 = {0};
    for (int i = 0; i < ITER; i++) {
        c0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c0, 0, 0, 0);
        c1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c1, 0, 0, 0);
        c2 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c2, 0, 0, 0);
        c3 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c3, 0, 0, 0);
    }
    int s = 0;
    for (int v = 0; v < 16; v++) s += c0[v] + c1[v] + c2[v] + c3[v];
    if (s == 0x12345678) out[0] = s;                  // keeps the chains live
}

__global__ __launch_bounds__(256) void k_mfma16(int seed, int *out) {
    const v4i a = {seed, seed + 1, seed + 2, seed + 3}, b = {seed ^ 5, seed ^ 7, seed ^ 9, seed ^ 11};
    v4i c0 = {0}, c1 = {0}, c2 = {0}, c3 = {0};
    for (int i = 0; i < ITER; i++) {
        c0 = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c0, 0, 0, 0);
        c1 = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c1, 0, 0, 0);
        c2 = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c2, 0, 0, 0);
        c3 = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c3, 0, 0, 0);
    }
    const int s = c0[0] + c1[1] + c2[2] + c3[3];
    if (s == 0x12345678) out[0] = s;
}

static double run(int kind, int *out) {
    hipEvent_t e0, e1;
    if (hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess) return -1;
    const int reps = 5;
    for (int r = -1; r < reps; r++) {                 // r = -1 warms up
        if (r == 0 && hipEventRecord(e0) != hipSuccess) return -1;
        if (kind == 0) hipLaunchKernelGGL(k_mfma32, dim3(GRID), dim3(256), 0, 0, 1, out);
        else hipLaunchKernelGGL(k_mfma16, dim3(GRID), dim3(256), 0, 0, 1, out);
        if (hipGetLastError() != hipSuccess) return -1;
    }
    float ms = 0;
    if (hipEventRecord(e1) != hipSuccess || hipEventSynchronize(e1) != hipSuccess ||
        hipEventElapsedTime(&ms, e0, e1) != hipSuccess)
        return -1;
    const double per_inst = kind == 0 ? 2.0 * 32 * 32 * 32 : 2.0 * 16 * 16 * 64;
    const double ops = (double)reps * GRID * 4 /*waves*/ * ITER * 4 /*chains*/ * per_inst;
    return ops / (ms * 1e-3) / 1e12;
}

int main(void) {
    int *out = nullptr;
    if (hipMalloc(&out, sizeof(int)) != hipSuccess) {
        fprintf(stderr, "mfma_peak: hipMalloc failed\n");
        return 1;
    }
    const double t32 = run(0, out), t16 = run(1, out);
    (void)hipFree(out);
    if (t32 < 0 || t16 < 0) {
        fprintf(stderr, "mfma_peak: HIP error\n");
        return 1;
    }
    printf("{\"mfma_i32_32x32x32_i8_tops\": %.1f, \"mfma_i32_16x16x64_i8_tops\": %.1f}\n", t32, t16);
    return 0;
}
