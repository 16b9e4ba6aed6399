// qk_api.cpp -- the C ABI of libqk (include/qk.h).
//
// Validates shapes and pointers on the host before any launch (every
// kernel assumes the shapes checked here), owns the library stream, the
// weight registry of the host seam and its scratch buffers, and picks
// the float-epilogue tier.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>
#include <unordered_map>

#if defined(__x86_64__) || defined(__i386__)
#include <cpuid.h>
#endif

#include "../../include/qk.h"
#include "qk_kernels.h"

namespace {

thread_local std::string g_err;

struct Weight {
    int type;
    int64_t k, n;
    size_t bytes;
    void *dev;
};

struct State {
    std::mutex mu;
    bool init = false;
    int device = -1;
    int tier = QK_TIER_SCALAR;
    hipStream_t stream = nullptr;
    std::string label;
    std::unordered_map<const void *, Weight> weights;
    // host-seam scratch (grown on demand)
    void *dx = nullptr;   size_t dx_cap = 0;
    void *dxq = nullptr;  size_t dxq_cap = 0;
    void *dy = nullptr;   size_t dy_cap = 0;
    void *dsel = nullptr; size_t dsel_cap = 0;
    // pinned host staging of the host seam: x goes in, y comes out
    void *hx = nullptr;   size_t hx_cap = 0;
    void *hy = nullptr;   size_t hy_cap = 0;
    int cu_count = 256;
};

State &st() {
    static State s;
    return s;
}

int fail(int code, const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_err = buf;
    return code;
}

int hip_fail(hipError_t e, const char *what) {
    return fail(QK_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

#define HIP_OK(expr, what)                          \
    do {                                            \
        hipError_t e_ = (expr);                     \
        if (e_ != hipSuccess) return hip_fail(e_, what); \
    } while (0)

// detect_cpu + simd_init tier selection, simd/simd.c:142-170,208-229.
int detect_tier() {
    int tier = QK_TIER_SCALAR;
#if defined(__x86_64__) || defined(__i386__)
    unsigned a = 0, b = 0, c = 0, d = 0;
    bool avx = false, fma = false, avx2 = false, vnni = false;
    if (__get_cpuid_count(1, 0, &a, &b, &c, &d)) {
        avx = (c >> 28) & 1;
        fma = (c >> 12) & 1;
    }
    if (__get_cpuid_count(7, 0, &a, &b, &c, &d)) avx2 = (b >> 5) & 1;
    if (__get_cpuid_count(7, 1, &a, &b, &c, &d)) vnni = (a >> 4) & 1;
    if (vnni && avx2 && fma) tier = QK_TIER_AVXVNNI;
    else if (avx2 && fma) tier = QK_TIER_AVX2;
    else if (avx) tier = QK_TIER_AVX1;
#endif
    return tier;
}

int fused_of(int tier) { return (tier == QK_TIER_AVX2 || tier == QK_TIER_AVXVNNI) ? 1 : 0; }

hipStream_t stream_of(void *s) { return reinterpret_cast<hipStream_t>(s); }

int64_t block_elems(int type) { return type == QK_TYPE_Q8_0 ? QK8_0 : QK_K; }

int64_t block_bytes(int type) {
    switch (type) {
        case QK_TYPE_Q8_0: return 34;
        case QK_TYPE_Q4_K: return 144;
        case QK_TYPE_Q5_K: return 176;
        case QK_TYPE_Q6_K: return 210;
        default: return 0;
    }
}

int64_t act_bytes(int type, int64_t k) {
    return type == QK_TYPE_Q8_0 ? (k / QK8_0) * 34 : (k / QK_K) * 292;
}

bool aligned(const void *p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }

int require_init() {
    if (!st().init) return fail(QK_ERR_NOT_INIT, "hip_qk_init has not succeeded");
    return QK_OK;
}

// Shape and alignment contract shared by every matvec/matmul entry point.
int check_mat(int type, const void *w, int64_t n, int64_t k, const void *xq, const void *y) {
    if (block_bytes(type) == 0) return fail(QK_ERR_UNSUPPORTED, "unsupported tensor type %d", type);
    if (!w || !xq || !y) return fail(QK_ERR_ARG, "null pointer");
    if (n < 1 || k < 1) return fail(QK_ERR_ARG, "empty matrix (n=%lld, k=%lld)", (long long)n, (long long)k);
    if (k % block_elems(type)) return fail(QK_ERR_ARG, "k=%lld is not a multiple of %lld", (long long)k, (long long)block_elems(type));
    if (k > 16384) return fail(QK_ERR_ARG, "k=%lld exceeds the 16384 limit", (long long)k);
    if (n > 0x7fffffffLL) return fail(QK_ERR_ARG, "n=%lld exceeds 2^31-1 rows", (long long)n);
    // The GEMV streams the matrix with 16-byte loads from its base and
    // addresses it with 32-bit byte offsets (buffer loads).
    if (!aligned(w, 16)) return fail(QK_ERR_ARG, "weights must be 16-byte aligned");
    const int64_t row_bytes = (k / block_elems(type)) * block_bytes(type);
    if (n * row_bytes > qk::gemv_max_matrix_bytes())
        return fail(QK_ERR_ARG, "matrix of %lld bytes exceeds the %lld-byte limit",
                    (long long)(n * row_bytes), (long long)qk::gemv_max_matrix_bytes());
    if (!aligned(xq, type == QK_TYPE_Q8_0 ? 2 : 4)) return fail(QK_ERR_ARG, "activations misaligned");
    if (!aligned(y, 4)) return fail(QK_ERR_ARG, "output misaligned");
    return QK_OK;
}

// Pinned host buffer of at least `need` bytes (contents not kept).
int grow_host(void **p, size_t *cap, size_t need) {
    if (*cap >= need) return QK_OK;
    if (*p) (void)hipHostFree(*p);
    *p = nullptr;
    *cap = 0;
    const size_t n = need < 65536 ? 65536 : need + need / 4;
    HIP_OK(hipHostMalloc(p, n, hipHostMallocDefault), "hipHostMalloc");
    *cap = n;
    return QK_OK;
}

int grow(void **p, size_t *cap, size_t need) {
    if (*cap >= need) return QK_OK;
    if (*p) (void)hipFree(*p);
    *p = nullptr;
    *cap = 0;
    size_t sz = need + need / 4 + 4096;
    HIP_OK(hipMalloc(p, sz), "hipMalloc(scratch)");
    *cap = sz;
    return QK_OK;
}

int matvec(int type, const void *w, int64_t n, int64_t k, const void *xq, float *y, void *s) {
    int rc = require_init();
    if (rc) return rc;
    if ((rc = check_mat(type, w, n, k, xq, y))) return rc;
    qk::GemvArgs a{};
    a.count = 1;
    a.fused = fused_of(st().tier);
    a.d[0].type = type;
    a.d[0].n = n;
    a.d[0].k = k;
    a.d[0].w = static_cast<const uint8_t *>(w);
    a.d[0].xq = static_cast<const uint8_t *>(xq);
    a.d[0].y = y;
    qk::gemv_plan(a.d[0]);
    HIP_OK(qk::launch_gemv(a, st().cu_count * 8, stream_of(s)), "gemv launch");
    return QK_OK;
}

int matmul(int type, const void *w, int64_t n, int64_t k, const void *xq, int64_t m, float *y, void *s) {
    int rc = require_init();
    if (rc) return rc;
    if ((rc = check_mat(type, w, n, k, xq, y))) return rc;
    if (m < 1 || m > 65535LL * 64) return fail(QK_ERR_ARG, "m=%lld tokens (1..%lld)", (long long)m, 65535LL * 64);
    if (type == QK_TYPE_Q8_0) return fail(QK_ERR_UNSUPPORTED, "no Q8_0 GEMM; use hip_matvec_q8_0 per token");
    HIP_OK(qk::launch_gemm(type, static_cast<const uint8_t *>(w), n, k,
                           static_cast<const uint8_t *>(xq), m, y, fused_of(st().tier), stream_of(s)),
           "gemm launch");
    return QK_OK;
}

}  // namespace

extern "C" {

int hip_qk_init(int device) {
    State &s = st();
    std::lock_guard<std::mutex> lk(s.mu);
    if (s.init && s.device == device) return QK_OK;
    int count = 0;
    HIP_OK(hipGetDeviceCount(&count), "hipGetDeviceCount");
    if (device < 0 || device >= count) return fail(QK_ERR_ARG, "device %d of %d", device, count);
    HIP_OK(hipSetDevice(device), "hipSetDevice");
    hipDeviceProp_t prop;
    HIP_OK(hipGetDeviceProperties(&prop, device), "hipGetDeviceProperties");
    if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
        return fail(QK_ERR_UNSUPPORTED, "libqk is built for gfx950, device is %s", prop.gcnArchName);
    if (!s.stream) HIP_OK(hipStreamCreateWithFlags(&s.stream, hipStreamNonBlocking), "hipStreamCreate");
    s.device = device;
    s.cu_count = prop.multiProcessorCount > 0 ? prop.multiProcessorCount : 256;
    s.tier = detect_tier();
    s.label = std::string(prop.gcnArchName) + " " + prop.name + " / tier " + hip_qk_tier_label(s.tier);
    s.init = true;
    return QK_OK;
}

void hip_qk_shutdown(void) {
    State &s = st();
    std::lock_guard<std::mutex> lk(s.mu);
    if (!s.init) return;
    (void)hipStreamSynchronize(s.stream);
    for (auto &kv : s.weights) (void)hipFree(kv.second.dev);
    s.weights.clear();
    void **bufs[] = {&s.dx, &s.dxq, &s.dy, &s.dsel};
    for (void **b : bufs) {
        if (*b) (void)hipFree(*b);
        *b = nullptr;
    }
    s.dx_cap = s.dxq_cap = s.dy_cap = s.dsel_cap = 0;
    void **hbufs[] = {&s.hx, &s.hy};
    for (void **b : hbufs) {
        if (*b) (void)hipHostFree(*b);
        *b = nullptr;
    }
    s.hx_cap = s.hy_cap = 0;
    (void)hipStreamDestroy(s.stream);
    s.stream = nullptr;
    s.init = false;
}

const char *hip_qk_device_label(void) { return st().init ? st().label.c_str() : "uninitialized"; }

const char *hip_qk_last_error(void) { return g_err.c_str(); }

const char *hip_qk_tier_label(int tier) {
    switch (tier) {
        case QK_TIER_AVX1: return "AVX1";
        case QK_TIER_AVX2: return "AVX2-FMA";
        case QK_TIER_AVXVNNI: return "AVX-VNNI";
        default: return "scalar";
    }
}

int hip_qk_set_tier(int tier) {
    if (tier == QK_TIER_AUTO) tier = detect_tier();
    if (tier < QK_TIER_SCALAR || tier > QK_TIER_AVXVNNI) return fail(QK_ERR_ARG, "tier %d", tier);
    st().tier = tier;
    return QK_OK;
}

int hip_qk_get_tier(void) { return st().tier; }

int hip_quantize_q8k(const float *x, int64_t m, int64_t k, void *xq, void *stream) {
    int rc = require_init();
    if (rc) return rc;
    if (!x || !xq) return fail(QK_ERR_ARG, "null pointer");
    if (m < 1 || k < 1 || k % QK_K) return fail(QK_ERR_ARG, "bad shape m=%lld k=%lld", (long long)m, (long long)k);
    if (!aligned(x, 16) || !aligned(xq, 4)) return fail(QK_ERR_ARG, "x must be 16-byte and xq 4-byte aligned");
    HIP_OK(qk::launch_quantize_q8k(x, m * (k / QK_K), static_cast<uint8_t *>(xq), stream_of(stream)),
           "quantize_q8k launch");
    return QK_OK;
}

int hip_quantize_q8_0(const float *x, int64_t m, int64_t k, void *xq, void *stream) {
    int rc = require_init();
    if (rc) return rc;
    if (!x || !xq) return fail(QK_ERR_ARG, "null pointer");
    if (m < 1 || k < 1 || k % QK8_0) return fail(QK_ERR_ARG, "bad shape m=%lld k=%lld", (long long)m, (long long)k);
    if (!aligned(x, 4) || !aligned(xq, 2)) return fail(QK_ERR_ARG, "misaligned x/xq");
    HIP_OK(qk::launch_quantize_q8_0(x, m * (k / QK8_0), static_cast<uint8_t *>(xq), stream_of(stream)),
           "quantize_q8_0 launch");
    return QK_OK;
}

int hip_matvec_q4k(const void *w, int64_t n, int64_t k, const void *xq, float *y, void *s) {
    return matvec(QK_TYPE_Q4_K, w, n, k, xq, y, s);
}
int hip_matvec_q5k(const void *w, int64_t n, int64_t k, const void *xq, float *y, void *s) {
    return matvec(QK_TYPE_Q5_K, w, n, k, xq, y, s);
}
int hip_matvec_q6k(const void *w, int64_t n, int64_t k, const void *xq, float *y, void *s) {
    return matvec(QK_TYPE_Q6_K, w, n, k, xq, y, s);
}
int hip_matvec_q8_0(const void *w, int64_t n, int64_t k, const void *xq, float *y, void *s) {
    return matvec(QK_TYPE_Q8_0, w, n, k, xq, y, s);
}

int hip_matvec_group(const qk_gemv_desc *desc, int count, void *stream) {
    int rc = require_init();
    if (rc) return rc;
    if (!desc || count < 1 || count > QK_GROUP_MAX)
        return fail(QK_ERR_ARG, "group count %d (1..%d)", count, QK_GROUP_MAX);
    qk::GemvArgs a{};
    a.count = count;
    a.fused = fused_of(st().tier);
    for (int i = 0; i < count; i++) {
        const qk_gemv_desc &d = desc[i];
        if ((rc = check_mat(d.type, d.w, d.n, d.k, d.xq, d.y))) {
            return fail(rc, "descriptor %d: %s", i, g_err.c_str());
        }
        a.d[i].type = d.type;
        a.d[i].n = d.n;
        a.d[i].k = d.k;
        a.d[i].w = static_cast<const uint8_t *>(d.w);
        a.d[i].xq = static_cast<const uint8_t *>(d.xq);
        a.d[i].y = d.y;
        qk::gemv_plan(a.d[i]);
    }
    HIP_OK(qk::launch_gemv(a, 1 << 20, stream_of(stream)), "gemv group launch");
    return QK_OK;
}

int hip_matmul_q4k(const void *w, int64_t n, int64_t k, const void *xq, int64_t m, float *y, void *s) {
    return matmul(QK_TYPE_Q4_K, w, n, k, xq, m, y, s);
}
int hip_matmul_q5k(const void *w, int64_t n, int64_t k, const void *xq, int64_t m, float *y, void *s) {
    return matmul(QK_TYPE_Q5_K, w, n, k, xq, m, y, s);
}
int hip_matmul_q6k(const void *w, int64_t n, int64_t k, const void *xq, int64_t m, float *y, void *s) {
    return matmul(QK_TYPE_Q6_K, w, n, k, xq, m, y, s);
}

static int dequant(int type, const void *w, int64_t nblocks, float *y, void *s) {
    int rc = require_init();
    if (rc) return rc;
    if (!w || !y || nblocks < 1) return fail(QK_ERR_ARG, "bad dequant arguments");
    if (!aligned(y, 16)) return fail(QK_ERR_ARG, "y must be 16-byte aligned");
    if (!aligned(w, 2)) return fail(QK_ERR_ARG, "w must be 2-byte aligned");
    HIP_OK(qk::launch_dequant(type, static_cast<const uint8_t *>(w), nblocks, y, stream_of(s)), "dequant launch");
    return QK_OK;
}
int hip_dequant_q4k(const void *w, int64_t nb, float *y, void *s) { return dequant(QK_TYPE_Q4_K, w, nb, y, s); }
int hip_dequant_q5k(const void *w, int64_t nb, float *y, void *s) { return dequant(QK_TYPE_Q5_K, w, nb, y, s); }
int hip_dequant_q6k(const void *w, int64_t nb, float *y, void *s) { return dequant(QK_TYPE_Q6_K, w, nb, y, s); }

}  // extern "C"

namespace {
// Body of the LM-head entry point; the caller holds st().mu.
int lmhead_locked(const void *w, int64_t n, int64_t k, const void *xq, int topk, float *logits,
                  int32_t *argmax, int32_t *topk_idx, float *topk_val, hipStream_t stream) {
    State &s = st();
    int rc;
    if (!argmax) return fail(QK_ERR_ARG, "argmax output is required");
    if (topk < 0 || topk > QK_TOPK_MAX || topk > n) return fail(QK_ERR_ARG, "topk=%d", topk);
    if (topk > 0 && (!topk_idx || !topk_val)) return fail(QK_ERR_ARG, "top-k outputs are required");
    // Logits always go to device memory: the caller's buffer, or scratch.
    const size_t sel = qk::lmhead_cand_bytes(n, topk);
    const size_t lbytes = logits ? 0 : (size_t)n * sizeof(float);
    if ((rc = grow(&s.dsel, &s.dsel_cap, sel + lbytes + 256))) return rc;
    float *lg = logits ? logits
                       : reinterpret_cast<float *>(static_cast<uint8_t *>(s.dsel) + ((sel + 255) & ~(size_t)255));
    if ((rc = check_mat(QK_TYPE_Q6_K, w, n, k, xq, lg))) return rc;
    HIP_OK(qk::launch_lmhead(static_cast<const uint8_t *>(w), n, k, static_cast<const uint8_t *>(xq), topk, lg,
                             argmax, topk_idx, topk_val, s.dsel, fused_of(s.tier), stream),
           "lmhead launch");
    return QK_OK;
}
}  // namespace

extern "C" {

int hip_lmhead_q6k_argmax_topk(const void *w, int64_t n, int64_t k, const void *xq, int topk,
                               float *logits, int32_t *argmax, int32_t *topk_idx, float *topk_val,
                               void *stream) {
    int rc = require_init();
    if (rc) return rc;
    std::lock_guard<std::mutex> lk(st().mu);
    return lmhead_locked(w, n, k, xq, topk, logits, argmax, topk_idx, topk_val, stream_of(stream));
}

// ---- host seam ---------------------------------------------------------------

int hip_qk_register_weight(const void *host_w, int type, int64_t k, int64_t n) {
    int rc = require_init();
    if (rc) return rc;
    if (!host_w) return fail(QK_ERR_ARG, "null weight");
    if (block_bytes(type) == 0) return fail(QK_ERR_UNSUPPORTED, "unsupported tensor type %d", type);
    if (k < 1 || n < 1 || k % block_elems(type)) return fail(QK_ERR_ARG, "bad weight shape");
    State &s = st();
    std::lock_guard<std::mutex> lk(s.mu);
    auto it = s.weights.find(host_w);
    if (it != s.weights.end()) {
        const Weight &w = it->second;
        if (w.type != type || w.k != k || w.n != n)
            return fail(QK_ERR_ARG, "weight %p re-registered with a different shape/type", host_w);
        return QK_OK;
    }
    Weight w{type, k, n, (size_t)(n * (k / block_elems(type)) * block_bytes(type)), nullptr};
    HIP_OK(hipMalloc(&w.dev, w.bytes), "hipMalloc(weight)");
    hipError_t e = hipMemcpy(w.dev, host_w, w.bytes, hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        (void)hipFree(w.dev);
        return hip_fail(e, "hipMemcpy(weight)");
    }
    s.weights.emplace(host_w, w);
    return QK_OK;
}

int hip_qk_unregister_weight(const void *host_w) {
    State &s = st();
    std::lock_guard<std::mutex> lk(s.mu);
    auto it = s.weights.find(host_w);
    if (it == s.weights.end()) return fail(QK_ERR_UNREGISTERED, "weight %p is not registered", host_w);
    (void)hipFree(it->second.dev);
    s.weights.erase(it);
    return QK_OK;
}

const void *hip_qk_device_weight(const void *host_w) {
    State &s = st();
    std::lock_guard<std::mutex> lk(s.mu);
    auto it = s.weights.find(host_w);
    return it == s.weights.end() ? nullptr : it->second.dev;
}

int hip_qk_matmul_host(const void *host_w, int type, int64_t out_f, int64_t k, const float *x,
                       int64_t n_tok, float *out) {
    int rc = require_init();
    if (rc) return rc;
    if (!x || !out || n_tok < 1) return fail(QK_ERR_ARG, "bad activation arguments");
    if ((rc = hip_qk_register_weight(host_w, type, k, out_f))) return rc;
    State &s = st();
    std::lock_guard<std::mutex> lk(s.mu);
    const Weight &w = s.weights.at(host_w);
    const size_t xb = (size_t)(n_tok * k) * sizeof(float);
    const size_t qb = (size_t)(n_tok * act_bytes(type, k));
    const size_t yb = (size_t)(n_tok * out_f) * sizeof(float);
    if ((rc = grow(&s.dx, &s.dx_cap, xb)) || (rc = grow(&s.dxq, &s.dxq_cap, qb)) ||
        (rc = grow(&s.dy, &s.dy_cap, yb)) || (rc = grow_host(&s.hx, &s.hx_cap, xb)) ||
        (rc = grow_host(&s.hy, &s.hy_cap, yb)))
        return rc;
    // x through pinned memory: a decode row (<= 16 KB) is read by the
    // quantizer straight from host memory; a prefill chunk goes by DMA.
    std::memcpy(s.hx, x, xb);
    void *hx_dev = nullptr;
    HIP_OK(hipHostGetDevicePointer(&hx_dev, s.hx, 0), "hipHostGetDevicePointer");
    const float *dx = static_cast<const float *>(hx_dev);
    if (xb > 16384) {
        HIP_OK(hipMemcpyAsync(s.dx, s.hx, xb, hipMemcpyHostToDevice, s.stream), "hipMemcpyAsync(x)");
        dx = static_cast<const float *>(s.dx);
    }
    uint8_t *dxq = static_cast<uint8_t *>(s.dxq);
    // y likewise: a small output (decode rows, <= 64 KB) is written by the
    // kernel straight into pinned host memory; a larger one goes by DMA.
    float *dy = static_cast<float *>(s.dy);
    const bool y_direct = yb <= 65536;
    if (y_direct) {
        void *hy_dev = nullptr;
        HIP_OK(hipHostGetDevicePointer(&hy_dev, s.hy, 0), "hipHostGetDevicePointer");
        dy = static_cast<float *>(hy_dev);
    }
    if (type == QK_TYPE_Q8_0) {
        HIP_OK(qk::launch_quantize_q8_0(dx, n_tok * (k / QK8_0), dxq, s.stream), "quantize");
        // tensor_matmul_q8_0_f32 has no batched form: up to 16 tokens per launch.
        for (int64_t t0 = 0; t0 < n_tok; t0 += QK_GROUP_MAX_DEV) {
            qk::GemvArgs a{};
            a.fused = fused_of(s.tier);
            a.count = (int32_t)((n_tok - t0) < QK_GROUP_MAX_DEV ? (n_tok - t0) : QK_GROUP_MAX_DEV);
            for (int i = 0; i < a.count; i++) {
                a.d[i].type = type;
                a.d[i].n = out_f;
                a.d[i].k = k;
                a.d[i].w = static_cast<const uint8_t *>(w.dev);
                a.d[i].xq = dxq + (t0 + i) * act_bytes(type, k);
                a.d[i].y = dy + (t0 + i) * out_f;
                qk::gemv_plan(a.d[i]);
            }
            HIP_OK(qk::launch_gemv(a, 1 << 20, s.stream), "gemv launch");
        }
    } else {
        HIP_OK(qk::launch_quantize_q8k(dx, n_tok * (k / QK_K), dxq, s.stream), "quantize");
        if (n_tok == 1) {
            qk::GemvArgs a{};
            a.fused = fused_of(s.tier);
            a.count = 1;
            a.d[0].type = type;
            a.d[0].n = out_f;
            a.d[0].k = k;
            a.d[0].w = static_cast<const uint8_t *>(w.dev);
            a.d[0].xq = dxq;
            a.d[0].y = dy;
            qk::gemv_plan(a.d[0]);
            HIP_OK(qk::launch_gemv(a, s.cu_count * 8, s.stream), "gemv launch");
        } else {
            HIP_OK(qk::launch_gemm(type, static_cast<const uint8_t *>(w.dev), out_f, k, dxq, n_tok, dy,
                                   fused_of(s.tier), s.stream),
                   "gemm launch");
        }
    }
    if (!y_direct)
        HIP_OK(hipMemcpyAsync(s.hy, dy, yb, hipMemcpyDeviceToHost, s.stream), "hipMemcpyAsync(out)");
    HIP_OK(hipStreamSynchronize(s.stream), "hipStreamSynchronize");
    std::memcpy(out, s.hy, yb);
    return QK_OK;
}

int hip_qk_lmhead_host(const void *host_w, int64_t n, int64_t k, const float *x, int topk,
                       float *logits, int32_t *argmax, int32_t *topk_idx, float *topk_val) {
    int rc = require_init();
    if (rc) return rc;
    if (!x || !argmax) return fail(QK_ERR_ARG, "bad arguments");
    if (topk < 0 || topk > QK_TOPK_MAX || topk > n) return fail(QK_ERR_ARG, "topk=%d", topk);
    if (topk > 0 && (!topk_idx || !topk_val)) return fail(QK_ERR_ARG, "top-k outputs are required");
    if ((rc = hip_qk_register_weight(host_w, QK_TYPE_Q6_K, k, n))) return rc;
    State &s = st();
    std::lock_guard<std::mutex> lk(s.mu);
    const void *wdev = s.weights.at(host_w).dev;
    const size_t xb = (size_t)k * sizeof(float);
    const size_t qb = (size_t)act_bytes(QK_TYPE_Q6_K, k);
    // dy: logits (n) | argmax (1) | topk idx (QK_TOPK_MAX) | topk val (QK_TOPK_MAX)
    const size_t yb = (size_t)(n + 1 + 2 * QK_TOPK_MAX) * sizeof(float) + 64;
    if ((rc = grow(&s.dx, &s.dx_cap, xb)) || (rc = grow(&s.dxq, &s.dxq_cap, qb)) ||
        (rc = grow(&s.dy, &s.dy_cap, yb)))
        return rc;
    HIP_OK(hipMemcpyAsync(s.dx, x, xb, hipMemcpyHostToDevice, s.stream), "hipMemcpyAsync(x)");
    HIP_OK(qk::launch_quantize_q8k(static_cast<const float *>(s.dx), k / QK_K, static_cast<uint8_t *>(s.dxq),
                                   s.stream),
           "quantize");
    float *dl = static_cast<float *>(s.dy);
    int32_t *dam = reinterpret_cast<int32_t *>(dl + n);
    int32_t *dti = dam + 1;
    float *dtv = reinterpret_cast<float *>(dti + QK_TOPK_MAX);
    if ((rc = lmhead_locked(wdev, n, k, s.dxq, topk, dl, dam, dti, dtv, s.stream))) return rc;
    if (logits)
        HIP_OK(hipMemcpyAsync(logits, dl, (size_t)n * sizeof(float), hipMemcpyDeviceToHost, s.stream), "copy logits");
    HIP_OK(hipMemcpyAsync(argmax, dam, sizeof(int32_t), hipMemcpyDeviceToHost, s.stream), "copy argmax");
    if (topk > 0) {
        HIP_OK(hipMemcpyAsync(topk_idx, dti, (size_t)topk * sizeof(int32_t), hipMemcpyDeviceToHost, s.stream),
               "copy topk idx");
        HIP_OK(hipMemcpyAsync(topk_val, dtv, (size_t)topk * sizeof(float), hipMemcpyDeviceToHost, s.stream),
               "copy topk val");
    }
    HIP_OK(hipStreamSynchronize(s.stream), "hipStreamSynchronize");
    return QK_OK;
}

}  // extern "C"
