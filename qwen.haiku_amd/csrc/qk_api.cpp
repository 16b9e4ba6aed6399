// qk_api.cpp -- the C ABI of libqk (include/qk.h).
//
// Validates shapes and pointers on the host before any launch (every
// kernel assumes the shapes checked here), owns the library stream, the
// weight registry of the host seam and its scratch buffers, and picks
// the float-epilogue tier.
#include <hip/hip_runtime.h>

#include <atomic>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <shared_mutex>
#include <string>
#include <unordered_map>
#include <vector>

#if defined(__x86_64__) || defined(__i386__)
#include <cpuid.h>
#endif

#include "../../include/qk.h"
#include "qk_kernels.h"

#include <cmath>
#define QK_EXPF_HOST 1                         // qk_expf on the host, for host_expf_ok
#include "qk_expf.h"

namespace {

thread_local std::string g_err;

struct Weight {
    int type;
    int64_t k, n;
    size_t bytes;
    void *dev;
    void *planes = nullptr;    // Q5_K / Q6_K: int8 MFMA planes, made at the first prefill GEMM
};

void free_weight(Weight &w) {
    (void)hipFree(w.dev);
    if (w.planes) (void)hipFree(w.planes);
    w.dev = w.planes = nullptr;
}

// Host-seam working set of one host thread: its own stream (the
// reference's contexts are single-threaded each, slm/slm.h:33-36, so a
// thread stands for a context), device scratch and pinned staging.
struct Lane {
    hipStream_t stream = nullptr;
    void *dx = nullptr;   size_t dx_cap = 0;
    void *dxq = nullptr;  size_t dxq_cap = 0;
    void *dy = nullptr;   size_t dy_cap = 0;
    void *dsel = nullptr; size_t dsel_cap = 0;
    void *hx = nullptr;   size_t hx_cap = 0;
    void *hy = nullptr;   size_t hy_cap = 0;
};

// Selection scratch (LM head, sampler) of one caller stream.
struct Sel {
    void *p = nullptr;
    size_t cap = 0;
};

struct State {
    std::mutex mu;                     // init/shutdown, lanes, sel, retired
    std::shared_mutex wmu;             // the weight registry
    bool init = false;
    int device = -1;
    std::atomic<int> tier{QK_TIER_SCALAR};
    std::atomic<uint64_t> gen{0};      // bumped by shutdown: thread-local lanes go stale
    std::string label;
    std::unordered_map<const void *, Weight> weights;
    std::vector<Lane *> lanes;
    std::unordered_map<hipStream_t, Sel> sel;
    // Scratch replaced by a larger one. Work already enqueued (or a
    // captured graph) may still point at it, so it is freed only at
    // shutdown.
    std::vector<void *> retired;
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

// Selection scratch of hip_lmhead_q6k_argmax_topk_noalloc: the argmax
// partials, candidate keys and counter, then (when the caller passes no
// logits buffer) up to QK_NOALLOC_MAX_N logits. One copy per GPU, held
// for the life of the process. Host code never uses this name as an
// address: hip_qk_init resolves each device's copy with
// hipGetSymbolAddress and the entry point passes that pointer.
constexpr size_t NOALLOC_SEL_BYTES = 40960;
constexpr size_t NOALLOC_SCRATCH_BYTES = NOALLOC_SEL_BYTES + (size_t)QK_NOALLOC_MAX_N * sizeof(float);
static __device__ __align__(256) uint8_t scratch[NOALLOC_SCRATCH_BYTES];
constexpr int MAX_DEVICES = 64;
void *g_noalloc[MAX_DEVICES];             // each device's `scratch`, set by hip_qk_init
// The last eager call of each device: its stream and an event recorded
// after it (created by hip_qk_init), so a call from another stream while
// that one is still in flight fails instead of racing on `scratch`.
std::mutex g_noalloc_mu;
hipEvent_t g_noalloc_ev[MAX_DEVICES];
hipStream_t g_noalloc_last[MAX_DEVICES];
bool g_noalloc_pending[MAX_DEVICES];

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

// The SiLU, softmax and DeltaNet gates of the reference call the host
// libm expf, and glibc picks one of two builds of it per CPU (fused
// multiply-adds on hosts with FMA and AVX2). The device implements the
// fused build (qk_expf.h). The builds differ on exactly two float inputs;
// this compares the host's expf with the restatement there, so it sees
// whichever build the process's libm dispatched to (tunables included).
bool host_expf_ok() {
    static const bool ok = [] {
        static const uint32_t probe[2] = {0x4202422fu, 0xc27c65d9u};
        for (uint32_t b : probe) {
            volatile uint32_t vb = b;                  // keep the compiler from folding expf
            float x;
            const uint32_t bb = vb;
            std::memcpy(&x, &bb, 4);
            const float h = std::exp(x), d = qk_expf(x);
            uint32_t hb, db;
            std::memcpy(&hb, &h, 4);
            std::memcpy(&db, &d, 4);
            if (hb != db) return false;
        }
        return true;
    }();
    return ok;
}

// Entry points whose kernels call expf: refused (before anything else,
// so the refusal shows on any host) when the host libm is the other build.
int require_host_expf(const char *what) {
    if (host_expf_ok()) return QK_OK;
    return fail(QK_ERR_UNSUPPORTED,
                "%s needs expf, and this host's libm expf is not the fused (FMA) build that the device "
                "reproduces: results would differ from the reference on this host",
                what);
}

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
    if (k > QK_MAX_K) return fail(QK_ERR_ARG, "k=%lld exceeds the %d limit", (long long)k, QK_MAX_K);
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

// Device scratch of at least `need` bytes (contents not kept). The old
// buffer is freed: only for buffers that no enqueued work still uses.
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

// The calling thread's current device is the library's. HIP's current
// device is per host thread, so a thread that reaches libqk first through
// a seam call or a scratch allocation selects it here once.
thread_local uint64_t t_dev_gen = ~0ull;

int ensure_device() {
    State &s = st();
    const uint64_t g = s.gen.load();
    if (t_dev_gen == g) return QK_OK;
    HIP_OK(hipSetDevice(s.device), "hipSetDevice");
    t_dev_gen = g;
    return QK_OK;
}

// The host-seam lane of the calling thread, created on its first call.
thread_local Lane *t_lane = nullptr;
thread_local uint64_t t_lane_gen = ~0ull;

int my_lane(Lane **out) {
    State &s = st();
    int rc;
    if ((rc = ensure_device())) return rc;
    if (t_lane && t_lane_gen == s.gen.load()) {
        *out = t_lane;
        return QK_OK;
    }
    Lane *l = new Lane();
    hipError_t e = hipStreamCreateWithFlags(&l->stream, hipStreamNonBlocking);
    if (e != hipSuccess) {
        delete l;
        return hip_fail(e, "hipStreamCreate(lane)");
    }
    {
        std::lock_guard<std::mutex> lk(s.mu);
        s.lanes.push_back(l);
    }
    t_lane = l;
    t_lane_gen = s.gen.load();
    *out = l;
    return QK_OK;
}

void free_lane(Lane *l) {
    (void)hipStreamSynchronize(l->stream);
    void *dev[] = {l->dx, l->dxq, l->dy, l->dsel};
    for (void *p : dev)
        if (p) (void)hipFree(p);
    void *hst[] = {l->hx, l->hy};
    for (void *p : hst)
        if (p) (void)hipHostFree(p);
    (void)hipStreamDestroy(l->stream);
    delete l;
}

// Workgroups of a single GEMV launch; a matrix with more tiles than that
// grid-strides over them. Measured on MI355X (graph replays, weights
// streamed from HBM): Q4_K is 4-8 % faster at 4 workgroups per CU than at
// 8 once it streams (248320x1024 24.5 -> 23.7 us, 65536x2048 15.3 ->
// 14.1 us), while Q6_K and Q8_0 are 1-4 % slower there, and 6 per CU is
// slower for every type.
int matvec_grid(int type) { return st().cu_count * (type == QK_TYPE_Q4_K ? 4 : 8); }

int matvec(int type, const void *w, int64_t n, int64_t k, const void *xq, float *y, void *s) {
    int rc = require_init();
    if (rc) return rc;
    if ((rc = check_mat(type, w, n, k, xq, y))) return rc;
    qk::GemvArgs a{};
    a.count = 1;
    a.fused = fused_of(st().tier.load());
    a.d[0].type = type;
    a.d[0].n = n;
    a.d[0].k = k;
    a.d[0].w = static_cast<const uint8_t *>(w);
    a.d[0].xq = static_cast<const uint8_t *>(xq);
    a.d[0].y = y;
    qk::gemv_plan(a.d[0]);
    HIP_OK(qk::launch_gemv(a, matvec_grid(type), stream_of(s)), "gemv launch");
    return QK_OK;
}

// Token bound of the GEMM: grid.y = token tiles of 64 (K-quants) or 32
// (Q8_0), at most 65535 of them.
int64_t gemm_max_m(int type) { return type == QK_TYPE_Q8_0 ? 65535LL * 32 : 65535LL * 64; }

int matmul(int type, const void *w, int64_t n, int64_t k, const void *xq, int64_t m, float *y, void *s) {
    int rc = require_init();
    if (rc) return rc;
    if ((rc = check_mat(type, w, n, k, xq, y))) return rc;
    if (m < 1 || m > gemm_max_m(type))
        return fail(QK_ERR_ARG, "m=%lld tokens (1..%lld)", (long long)m, (long long)gemm_max_m(type));
    HIP_OK(qk::launch_gemm(type, static_cast<const uint8_t *>(w), n, k, static_cast<const uint8_t *>(xq), m, y,
                           fused_of(st().tier.load()), stream_of(s)),
           "gemm launch");
    return QK_OK;
}

}  // namespace

extern "C" {

int hip_qk_init(int device) {
    State &s = st();
    std::lock_guard<std::mutex> lk(s.mu);
    if (s.init) {
        if (s.device == device) return QK_OK;
        return fail(QK_ERR_ARG, "libqk is initialized on device %d; hip_qk_shutdown first", s.device);
    }
    int count = 0;
    HIP_OK(hipGetDeviceCount(&count), "hipGetDeviceCount");
    if (device < 0 || device >= count) return fail(QK_ERR_ARG, "device %d of %d", device, count);
    HIP_OK(hipSetDevice(device), "hipSetDevice");
    hipDeviceProp_t prop;
    HIP_OK(hipGetDeviceProperties(&prop, device), "hipGetDeviceProperties");
    if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
        return fail(QK_ERR_UNSUPPORTED, "libqk is built for gfx950, device is %s", prop.gcnArchName);
    if (device < MAX_DEVICES && !g_noalloc[device]) {
        void *p = nullptr;
        HIP_OK(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)");
        HIP_OK(hipEventCreateWithFlags(&g_noalloc_ev[device], hipEventDisableTiming), "hipEventCreate(noalloc)");
        g_noalloc[device] = p;
    }
    s.device = device;
    s.cu_count = prop.multiProcessorCount > 0 ? prop.multiProcessorCount : 256;
    s.tier.store(detect_tier());
    char label[512];
    snprintf(label, sizeof label, "%s %s / tier %s", prop.gcnArchName, prop.name, hip_qk_tier_label(s.tier.load()));
    s.label = label;
    s.gen.fetch_add(1);
    t_dev_gen = s.gen.load();
    s.init = true;
    return QK_OK;
}

void hip_qk_shutdown(void) {
    State &s = st();
    std::lock_guard<std::mutex> lk(s.mu);
    if (!s.init) return;
    std::unique_lock<std::shared_mutex> wl(s.wmu);
    (void)hipSetDevice(s.device);
    (void)hipDeviceSynchronize();
    for (Lane *l : s.lanes) free_lane(l);
    s.lanes.clear();
    for (auto &kv : s.sel) (void)hipFree(kv.second.p);
    s.sel.clear();
    for (void *p : s.retired) (void)hipFree(p);
    s.retired.clear();
    for (auto &kv : s.weights) free_weight(kv.second);
    s.weights.clear();
    s.gen.fetch_add(1);                    // every thread's lane and device choice are stale
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
    st().tier.store(tier);
    return QK_OK;
}

int hip_qk_get_tier(void) { return st().tier.load(); }

int hip_quantize_q8k(const float *x, int64_t m, int64_t k, void *xq, void *stream) {
    int rc = require_init();
    if (rc) return rc;
    if (!x || !xq) return fail(QK_ERR_ARG, "null pointer");
    // a dispatch counts its work-items in 32 bits: 64 per block
    if (m < 1 || k < 1 || k % QK_K || m > ((int64_t)1 << 26) / (k / QK_K))
        return fail(QK_ERR_ARG, "bad shape m=%lld k=%lld (k a multiple of 256, m*k/256 at most 2^26)", (long long)m,
                    (long long)k);
    if (!aligned(x, 16) || !aligned(xq, 4)) return fail(QK_ERR_ARG, "x must be 16-byte and xq 4-byte aligned");
    HIP_OK(qk::launch_quantize_q8k(x, m * (k / QK_K), static_cast<uint8_t *>(xq), stream_of(stream)),
           "quantize_q8k launch");
    return QK_OK;
}

int hip_quantize_q8_0(const float *x, int64_t m, int64_t k, void *xq, void *stream) {
    int rc = require_init();
    if (rc) return rc;
    if (!x || !xq) return fail(QK_ERR_ARG, "null pointer");
    // a dispatch counts its work-items in 32 bits: 32 per block
    if (m < 1 || k < 1 || k % QK8_0 || m > ((int64_t)1 << 27) / (k / QK8_0))
        return fail(QK_ERR_ARG, "bad shape m=%lld k=%lld (k a multiple of 32, m*k/32 at most 2^27)", (long long)m,
                    (long long)k);
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
    a.fused = fused_of(st().tier.load());
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

int hip_matvec_group_f32(const qk_gemv_desc_f32 *desc, int count, void *stream) {
    int rc = require_init();
    if (rc) return rc;
    if (!desc || count < 1 || count > QK_GROUP_MAX)
        return fail(QK_ERR_ARG, "group count %d (1..%d)", count, QK_GROUP_MAX);
    qk::GemvArgs a{};
    a.count = count;
    a.fused = fused_of(st().tier.load());
    for (int i = 0; i < count; i++) {
        const qk_gemv_desc_f32 &d = desc[i];
        if ((rc = check_mat(d.type, d.w, d.n, d.k, d.x, d.y))) return fail(rc, "descriptor %d: %s", i, g_err.c_str());
        // the workgroups read the row with 16-byte (Q8_K) or 4-byte (Q8_0) loads
        if (!aligned(d.x, d.type == QK_TYPE_Q8_0 ? 4 : 16))
            return fail(QK_ERR_ARG, "descriptor %d: x must be %d-byte aligned", i, d.type == QK_TYPE_Q8_0 ? 4 : 16);
        a.d[i].type = d.type;
        a.d[i].n = d.n;
        a.d[i].k = d.k;
        a.d[i].w = static_cast<const uint8_t *>(d.w);
        a.d[i].xq = reinterpret_cast<const uint8_t *>(d.x);
        a.d[i].y = d.y;
        a.d[i].xf32 = 1;
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
int hip_matmul_q8_0(const void *w, int64_t n, int64_t k, const void *xq, int64_t m, float *y, void *s) {
    return matmul(QK_TYPE_Q8_0, w, n, k, xq, m, y, s);
}

size_t hip_gemm_planes_bytes(int type, int64_t n, int64_t k) {
    if (type != QK_TYPE_Q4_K && type != QK_TYPE_Q5_K && type != QK_TYPE_Q6_K) return 0;
    if (n < 1 || k < 1 || k % QK_K || k > QK_MAX_K || n > 0x7fffffffLL) return 0;
    return qk::gemm_planes_bytes(type, n, k);
}

int hip_gemm_pack_planes(int type, const void *w, int64_t n, int64_t k, void *planes, void *s) {
    int rc = require_init();
    if (rc) return rc;
    if (hip_gemm_planes_bytes(type, n, k) == 0)
        return fail(QK_ERR_UNSUPPORTED, "no planes for type %d, n=%lld, k=%lld", type, (long long)n, (long long)k);
    if ((rc = check_mat(type, w, n, k, planes, planes))) return rc;
    if (!aligned(planes, 16)) return fail(QK_ERR_ARG, "planes must be 16-byte aligned");
    const uintptr_t a = reinterpret_cast<uintptr_t>(w), b = reinterpret_cast<uintptr_t>(planes);
    const size_t wb = (size_t)n * (size_t)(k / QK_K) * block_bytes(type), pb = qk::gemm_planes_bytes(type, n, k);
    if (a < b + pb && b < a + wb) return fail(QK_ERR_ARG, "planes overlap the weights");
    HIP_OK(qk::launch_pack_planes(type, static_cast<const uint8_t *>(w), n, k, static_cast<uint8_t *>(planes),
                                  stream_of(s)),
           "pack launch");
    return QK_OK;
}

int hip_matmul_planes(int type, const void *planes, int64_t n, int64_t k, const void *xq, int64_t m, float *y,
                      void *s) {
    int rc = require_init();
    if (rc) return rc;
    if (hip_gemm_planes_bytes(type, n, k) == 0)
        return fail(QK_ERR_UNSUPPORTED, "no planes for type %d, n=%lld, k=%lld", type, (long long)n, (long long)k);
    if ((rc = check_mat(type, planes, n, k, xq, y))) return rc;
    if (m < 1 || m > gemm_max_m(type))
        return fail(QK_ERR_ARG, "m=%lld tokens (1..%lld)", (long long)m, (long long)gemm_max_m(type));
    HIP_OK(qk::launch_gemm_planes(type, static_cast<const uint8_t *>(planes), n, k, static_cast<const uint8_t *>(xq),
                                  m, y, fused_of(st().tier.load()), stream_of(s)),
           "gemm launch");
    return QK_OK;
}

static int dequant(int type, const void *w, int64_t nblocks, float *y, void *s) {
    int rc = require_init();
    if (rc) return rc;
    if (!w || !y || nblocks < 1 || nblocks > ((int64_t)1 << 26))   // 64 work-items per block, 32-bit count
        return fail(QK_ERR_ARG, "bad dequant arguments (nblocks 1..2^26)");
    if (!aligned(y, 16)) return fail(QK_ERR_ARG, "y must be 16-byte aligned");
    if (!aligned(w, 2)) return fail(QK_ERR_ARG, "w must be 2-byte aligned");
    HIP_OK(qk::launch_dequant(type, static_cast<const uint8_t *>(w), nblocks, y, stream_of(s)), "dequant launch");
    return QK_OK;
}
int hip_dequant_q4k(const void *w, int64_t nb, float *y, void *s) { return dequant(QK_TYPE_Q4_K, w, nb, y, s); }
int hip_dequant_q5k(const void *w, int64_t nb, float *y, void *s) { return dequant(QK_TYPE_Q5_K, w, nb, y, s); }
int hip_dequant_q6k(const void *w, int64_t nb, float *y, void *s) { return dequant(QK_TYPE_Q6_K, w, nb, y, s); }

int hip_add_rmsnorm_q8k(const float *h, const float *delta, const float *w, float eps, int64_t m, int64_t k,
                        float *h_out, float *x_out, void *xq, void *stream) {
    int rc = require_init();
    if (rc) return rc;
    if (!h || !w) return fail(QK_ERR_ARG, "null pointer");
    if (!x_out && !xq) return fail(QK_ERR_ARG, "x_out and xq are both NULL");
    // one 256-thread workgroup per row; a dispatch counts work-items in 32 bits
    if (m < 1 || m >= ((int64_t)1 << 24) || k < 4 || k % 4 || k > QK_NORM_MAX_K)
        return fail(QK_ERR_ARG, "bad shape m=%lld k=%lld (m below 2^24, k a multiple of 4, at most %d)",
                    (long long)m, (long long)k, QK_NORM_MAX_K);
    if (xq && k % QK_K) return fail(QK_ERR_ARG, "k=%lld: a Q8_K row needs a multiple of 256", (long long)k);
    if (!aligned(h, 16) || !aligned(delta, 16) || !aligned(w, 16) || !aligned(h_out, 16) || !aligned(x_out, 16) ||
        !aligned(xq, 4))
        return fail(QK_ERR_ARG, "float rows must be 16-byte and xq 4-byte aligned");
    if (delta == h_out && delta) return fail(QK_ERR_ARG, "h_out may alias h, not delta");
    HIP_OK(qk::launch_add_rmsnorm(h, delta, w, eps, m, k, h_out, x_out, static_cast<uint8_t *>(xq),
                                  stream_of(stream)),
           "add_rmsnorm launch");
    return QK_OK;
}

int hip_silu_f32(const float *x, int64_t n, float *y, void *stream) {
    int rc = require_host_expf("hip_silu_f32");
    if (rc) return rc;
    rc = require_init();
    if (rc) return rc;
    if (!x || !y || n < 1) return fail(QK_ERR_ARG, "bad silu arguments");
    if (!aligned(x, 4) || !aligned(y, 4)) return fail(QK_ERR_ARG, "x/y misaligned");
    HIP_OK(qk::launch_silu(x, y, n, stream_of(stream)), "silu launch");
    return QK_OK;
}

int hip_swiglu_q8k(const float *gate, const float *up, int64_t m, int64_t k, float *act, void *xq, void *stream) {
    int rc = require_host_expf("hip_swiglu_q8k");
    if (rc) return rc;
    rc = require_init();
    if (rc) return rc;
    if (!gate || !up) return fail(QK_ERR_ARG, "null pointer");
    if (!act && !xq) return fail(QK_ERR_ARG, "act and xq are both NULL");
    if (m < 1 || k < 4 || k % 4 || m > ((int64_t)1 << 33) / k)    // one wave per 256 elements
        return fail(QK_ERR_ARG, "bad shape m=%lld k=%lld (k a multiple of 4, m*k at most 2^33)", (long long)m,
                    (long long)k);
    if (xq && k % QK_K) return fail(QK_ERR_ARG, "k=%lld: a Q8_K row needs a multiple of 256", (long long)k);
    if (!aligned(gate, 16) || !aligned(up, 16) || !aligned(act, 16) || !aligned(xq, 4))
        return fail(QK_ERR_ARG, "float rows must be 16-byte and xq 4-byte aligned");
    HIP_OK(qk::launch_swiglu(gate, up, m * k, act, static_cast<uint8_t *>(xq), stream_of(stream)),
           "swiglu launch");
    return QK_OK;
}

}  // extern "C"

namespace {

int check_lmhead_outputs(int64_t n, int topk, const int32_t *argmax, const int32_t *topk_idx,
                         const float *topk_val) {
    if (!argmax) return fail(QK_ERR_ARG, "argmax output is required");
    if (topk < 0 || topk > QK_TOPK_MAX || topk > n) return fail(QK_ERR_ARG, "topk=%d", topk);
    if (topk > 0 && (!topk_idx || !topk_val)) return fail(QK_ERR_ARG, "top-k outputs are required");
    return QK_OK;
}

// LM head on `stream` with selection scratch `scratch` (at least
// lmhead_cand_bytes(n, topk) bytes, plus n floats of logits when `logits`
// is NULL, placed at the first 256-byte boundary past the selection part).
int lmhead_launch(const void *w, int64_t n, int64_t k, const void *xq, int topk, float *logits, int32_t *argmax,
                  int32_t *topk_idx, float *topk_val, void *scratch, hipStream_t stream) {
    int rc;
    const size_t sel = qk::lmhead_cand_bytes(n, topk);
    float *lg = logits ? logits
                       : reinterpret_cast<float *>(static_cast<uint8_t *>(scratch) + ((sel + 255) & ~(size_t)255));
    if ((rc = check_mat(QK_TYPE_Q6_K, w, n, k, xq, lg))) return rc;
    HIP_OK(qk::launch_lmhead(static_cast<const uint8_t *>(w), n, k, static_cast<const uint8_t *>(xq), topk, lg,
                             argmax, topk_idx, topk_val, scratch, fused_of(st().tier.load()), stream),
           "lmhead launch");
    return QK_OK;
}

size_t lmhead_scratch_bytes(int64_t n, int topk, bool own_logits) {
    const size_t sel = qk::lmhead_cand_bytes(n, topk);
    return ((sel + 255) & ~(size_t)255) + (own_logits ? (size_t)n * sizeof(float) : 0);
}

// Selection scratch of `stream` with room for `need` bytes. A stream keeps
// one buffer; a larger request replaces it and retires the old one, which
// earlier launches on the stream (or a graph captured from them) may still
// use, so it stays allocated until hip_qk_shutdown. Two streams never
// share a buffer.
int stream_scratch(hipStream_t stream, size_t need, void **out) {
    State &s = st();
    int rc;
    if ((rc = ensure_device())) return rc;
    std::lock_guard<std::mutex> lk(s.mu);
    Sel &e = s.sel[stream];
    if (e.cap < need) {
        // An allocation would invalidate a graph capture under way on the
        // stream: refuse instead, before anything is enqueued.
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        if (hipStreamIsCapturing(stream, &cs) == hipSuccess && cs != hipStreamCaptureStatusNone)
            return fail(QK_ERR_ARG,
                        "selection scratch for this stream must grow to %zu bytes, which allocates, and the "
                        "stream is capturing: make one call of this size on the stream before capture (for the "
                        "LM head, or use hip_lmhead_q6k_argmax_topk_noalloc)",
                        need);
        const size_t sz = need + need / 4 + 4096;
        void *p = nullptr;
        HIP_OK(hipMalloc(&p, sz), "hipMalloc(selection scratch)");
        if (e.p) s.retired.push_back(e.p);
        e.p = p;
        e.cap = sz;
    }
    *out = e.p;
    return QK_OK;
}

// Host buffers in and out: q | k | v | g | beta | state staged in this
// thread's pinned buffer, one copy each way, the launch on its stream,
// synchronous. State and out come back in one copy (they are adjacent on
// the device).
int deltanet_host(int64_t n_tok, int H, int k_hd, int v_hd, const float *q, const float *k, const float *v,
                  const float *g_log, const float *beta, float *state, float *out) {
    int rc;
    Lane *l = nullptr;
    if ((rc = my_lane(&l))) return rc;
    const size_t nq = (size_t)n_tok * H * k_hd, nv = (size_t)n_tok * H * v_hd, ng = (size_t)n_tok * H;
    const size_t ns = (size_t)H * k_hd * v_hd;
    const size_t in_floats = 2 * nq + nv + 2 * ng + ns;
    const size_t all = (in_floats + nv) * sizeof(float);
    if ((rc = grow(&l->dx, &l->dx_cap, all)) || (rc = grow_host(&l->hx, &l->hx_cap, all))) return rc;
    float *h = static_cast<float *>(l->hx);
    std::memcpy(h, q, nq * 4);
    std::memcpy(h + nq, k, nq * 4);
    std::memcpy(h + 2 * nq, v, nv * 4);
    std::memcpy(h + 2 * nq + nv, g_log, ng * 4);
    std::memcpy(h + 2 * nq + nv + ng, beta, ng * 4);
    std::memcpy(h + 2 * nq + nv + 2 * ng, state, ns * 4);
    float *d = static_cast<float *>(l->dx);
    HIP_OK(hipMemcpyAsync(d, h, in_floats * 4, hipMemcpyHostToDevice, l->stream), "hipMemcpyAsync(deltanet in)");
    void *scratch = nullptr;
    if ((rc = stream_scratch(l->stream, qk::deltanet_scratch_bytes(H, k_hd, v_hd, n_tok), &scratch))) return rc;
    float *dstate = d + 2 * nq + nv + 2 * ng, *dout = d + in_floats;
    HIP_OK(qk::launch_deltanet(d, d + nq, d + 2 * nq, d + 2 * nq + nv, d + 2 * nq + nv + ng, n_tok, H, k_hd, v_hd,
                               dstate, dout, scratch, l->stream),
           "deltanet launch");
    HIP_OK(hipMemcpyAsync(h + 2 * nq + nv + 2 * ng, dstate, (ns + nv) * 4, hipMemcpyDeviceToHost, l->stream),
           "hipMemcpyAsync(deltanet out)");
    HIP_OK(hipStreamSynchronize(l->stream), "hipStreamSynchronize");
    std::memcpy(state, h + 2 * nq + nv + 2 * ng, ns * 4);
    std::memcpy(out, h + in_floats, nv * 4);
    return QK_OK;
}

}  // namespace

extern "C" {

int hip_lmhead_q6k_argmax_topk(const void *w, int64_t n, int64_t k, const void *xq, int topk,
                               float *logits, int32_t *argmax, int32_t *topk_idx, float *topk_val,
                               void *stream) {
    int rc = require_init();
    if (rc) return rc;
    if ((rc = check_lmhead_outputs(n, topk, argmax, topk_idx, topk_val))) return rc;
    if (n < 1) return fail(QK_ERR_ARG, "empty matrix (n=%lld)", (long long)n);
    void *scratch = nullptr;
    if ((rc = stream_scratch(stream_of(stream), lmhead_scratch_bytes(n, topk, logits == nullptr), &scratch)))
        return rc;
    return lmhead_launch(w, n, k, xq, topk, logits, argmax, topk_idx, topk_val, scratch, stream_of(stream));
}

int hip_sample(float *logits, int64_t n, const qk_sampler *sp, uint64_t *rng, const int32_t *history,
               int32_t hist_n, const int32_t *mask, int32_t n_mask, int32_t *token, void *stream) {
    int rc;
    // the softmax of every non-greedy pick (a NaN temperature is not
    // greedy, slm/sampler.c:140) exponentiates
    if (sp && !(sp->temperature <= 0.0f) && (rc = require_host_expf("hip_sample"))) return rc;
    if ((rc = require_init())) return rc;
    if (!logits || !sp || !token) return fail(QK_ERR_ARG, "null pointer");
    if (n < 1 || n > QK_SAMPLE_MAX_N) return fail(QK_ERR_ARG, "n=%lld logits (1..%d)", (long long)n, QK_SAMPLE_MAX_N);
    if (hist_n < 0 || (hist_n > 0 && !history)) return fail(QK_ERR_ARG, "history of %d tokens", hist_n);
    if (n_mask < 0 || n_mask > QK_SAMPLE_MAX_MASK || (n_mask > 0 && !mask))
        return fail(QK_ERR_ARG, "n_mask=%d (0..%d)", n_mask, QK_SAMPLE_MAX_MASK);
    if (!(sp->temperature <= 0.0f) && (!rng || !aligned(rng, 8)))
        return fail(QK_ERR_ARG, "sampling (temperature > 0 or NaN) needs the 8-byte aligned rng state");
    if (!aligned(logits, 4) || !aligned(token, 4) || !aligned(history, 4))
        return fail(QK_ERR_ARG, "misaligned logits/token/history");
    int32_t k = sp->top_k > 0 ? sp->top_k : QK_TOPK_MAX;    // slm/sampler.c:143-144
    if (k > QK_TOPK_MAX) k = QK_TOPK_MAX;
    void *scratch = nullptr;
    if ((rc = stream_scratch(stream_of(stream), qk::sample_scratch_bytes(n, k), &scratch))) return rc;
    HIP_OK(qk::launch_sample(logits, n, sp->temperature, k, sp->top_p, sp->min_p, sp->repetition_penalty,
                             sp->repetition_window, rng, history, hist_n, mask, n_mask, token, scratch,
                             stream_of(stream)),
           "sample launch");
    return QK_OK;
}

int hip_deltanet_chunked(const float *q, const float *k, const float *v, const float *g_log, const float *beta,
                         int64_t n_tok, int n_heads, int k_hd, int v_hd, float *state, float *out, void *stream) {
    int rc = require_host_expf("hip_deltanet_chunked");
    if (rc) return rc;
    rc = require_init();
    if (rc) return rc;
    if (!q || !k || !v || !g_log || !beta || !state || !out) return fail(QK_ERR_ARG, "null pointer");
    if (n_tok < 1 || n_tok > 0x7fffffffLL || n_heads < 1 || n_heads > 1024 || k_hd < 1 || v_hd < 1 ||
        k_hd > QK_DELTANET_MAX_HD || v_hd > QK_DELTANET_MAX_HD)
        return fail(QK_ERR_ARG, "bad shape n_tok=%lld heads=%d k_hd=%d v_hd=%d (head dims 1..%d)", (long long)n_tok,
                    n_heads, k_hd, v_hd, QK_DELTANET_MAX_HD);
    if (!aligned(q, 4) || !aligned(k, 4) || !aligned(v, 4) || !aligned(g_log, 4) || !aligned(beta, 4) ||
        !aligned(state, 4) || !aligned(out, 4))
        return fail(QK_ERR_ARG, "misaligned float arrays");
    {   // out and the state are written while later phases and other
        // workgroups still read the inputs (and out, the state)
        const size_t nq = (size_t)n_tok * n_heads * k_hd * 4, nv = (size_t)n_tok * n_heads * v_hd * 4;
        const size_t ng = (size_t)n_tok * n_heads * 4, ns = (size_t)n_heads * k_hd * v_hd * 4;
        auto overlap = [](const void *o, size_t no, const void *a, size_t na) {
            const uintptr_t x = reinterpret_cast<uintptr_t>(o), y = reinterpret_cast<uintptr_t>(a);
            return x < y + na && y < x + no;
        };
        auto hits_input = [&](const void *o, size_t no) {
            return overlap(o, no, q, nq) || overlap(o, no, k, nq) || overlap(o, no, v, nv) ||
                   overlap(o, no, g_log, ng) || overlap(o, no, beta, ng);
        };
        if (hits_input(out, nv) || overlap(out, nv, state, ns))
            return fail(QK_ERR_ARG, "out overlaps an input or the state");
        if (hits_input(state, ns)) return fail(QK_ERR_ARG, "state overlaps an input");
    }
    void *scratch = nullptr;
    if ((rc = stream_scratch(stream_of(stream), qk::deltanet_scratch_bytes(n_heads, k_hd, v_hd, n_tok), &scratch)))
        return rc;
    HIP_OK(qk::launch_deltanet(q, k, v, g_log, beta, n_tok, n_heads, k_hd, v_hd, state, out, scratch,
                               stream_of(stream)),
           "deltanet launch");
    return QK_OK;
}

int hip_lmhead_q6k_argmax_topk_noalloc(const void *w, int64_t n, int64_t k, const void *xq, int topk,
                                       float *logits, int32_t *argmax, int32_t *topk_idx, float *topk_val,
                                       void *stream) {
    int rc = require_init();
    if (rc) return rc;
    if ((rc = check_lmhead_outputs(n, topk, argmax, topk_idx, topk_val))) return rc;
    if (n < 1) return fail(QK_ERR_ARG, "empty matrix (n=%lld)", (long long)n);
    const int dev = st().device;
    void *p = dev < MAX_DEVICES ? g_noalloc[dev] : nullptr;
    if (!p) return fail(QK_ERR_UNSUPPORTED, "no static scratch on device %d", dev);
    if (!logits && n > QK_NOALLOC_MAX_N)
        return fail(QK_ERR_ARG, "n=%lld rows without a logits buffer exceeds the static scratch (%d rows)",
                    (long long)n, QK_NOALLOC_MAX_N);
    if (lmhead_scratch_bytes(n, topk, logits == nullptr) > NOALLOC_SCRATCH_BYTES ||
        qk::lmhead_cand_bytes(n, topk) > NOALLOC_SEL_BYTES)
        return fail(QK_ERR_ARG, "static scratch too small for n=%lld", (long long)n);
    // Every call on this GPU shares `scratch`. An eager call from another
    // stream than the last one, while the last one is still in flight,
    // would race on it: refused. (Calls captured into a graph are not
    // tracked; their replays must be ordered by the caller.)
    const hipStream_t sm = stream_of(stream);
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    const bool capturing = hipStreamIsCapturing(sm, &cs) == hipSuccess && cs != hipStreamCaptureStatusNone;
    std::lock_guard<std::mutex> lk(g_noalloc_mu);
    if (!capturing && g_noalloc_pending[dev] && g_noalloc_last[dev] != sm &&
        hipEventQuery(g_noalloc_ev[dev]) == hipErrorNotReady)
        return fail(QK_ERR_ARG,
                    "the previous allocation-free LM head call on this GPU, on another stream, is still in flight: "
                    "both share one static scratch array; order the calls or keep them on one stream");
    // the kernels clear their own counter; nothing else must start at zero
    if ((rc = lmhead_launch(w, n, k, xq, topk, logits, argmax, topk_idx, topk_val, p, sm))) return rc;
    if (!capturing) {
        HIP_OK(hipEventRecord(g_noalloc_ev[dev], sm), "hipEventRecord(noalloc)");
        g_noalloc_last[dev] = sm;
        g_noalloc_pending[dev] = true;
    }
    return QK_OK;
}

}  // extern "C"

// ---- host seam ---------------------------------------------------------------

// Helpers of the seam entry points: C++ linkage and internal to this
// file, so libqk exports none of their names into the host process.
namespace {
// Caller holds s.wmu exclusively.
int register_locked(const void *host_w, int type, int64_t k, int64_t n) {
    State &s = st();
    auto it = s.weights.find(host_w);
    if (it != s.weights.end()) {
        const Weight &w = it->second;
        if (w.type != type || w.k != k || w.n != n)
            return fail(QK_ERR_ARG, "weight %p re-registered with a different shape/type", host_w);
        return QK_OK;
    }
    Weight w{type, k, n, (size_t)(n * (k / block_elems(type)) * block_bytes(type)), nullptr, nullptr};
    HIP_OK(hipMalloc(&w.dev, w.bytes), "hipMalloc(weight)");
    hipError_t e = hipMemcpy(w.dev, host_w, w.bytes, hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        (void)hipFree(w.dev);
        return hip_fail(e, "hipMemcpy(weight)");
    }
    s.weights.emplace(host_w, w);
    return QK_OK;
}

int check_weight_args(const void *host_w, int type, int64_t k, int64_t n) {
    if (!host_w) return fail(QK_ERR_ARG, "null weight");
    if (block_bytes(type) == 0) return fail(QK_ERR_UNSUPPORTED, "unsupported tensor type %d", type);
    if (k < 1 || n < 1 || k % block_elems(type) || k > QK_MAX_K || n > 0x7fffffffLL)
        return fail(QK_ERR_ARG, "bad weight shape n=%lld k=%lld", (long long)n, (long long)k);
    return QK_OK;
}

// Look up the device copy of `host_w` under the registry's shared lock,
// which the caller keeps for as long as it uses the copy, registering it
// first (exclusive lock) when it is new. On success `rl` holds the lock.
int acquire_weight(const void *host_w, int type, int64_t k, int64_t n, std::shared_lock<std::shared_mutex> &rl,
                   Weight *out) {
    State &s = st();
    int rc;
    for (int attempt = 0; attempt < 2; attempt++) {
        rl = std::shared_lock<std::shared_mutex>(s.wmu);
        auto it = s.weights.find(host_w);
        if (it != s.weights.end()) {
            const Weight &w = it->second;
            if (w.type != type || w.k != k || w.n != n)
                return fail(QK_ERR_ARG, "weight %p registered with a different shape/type", host_w);
            *out = w;
            return QK_OK;
        }
        rl.unlock();
        std::unique_lock<std::shared_mutex> wl(s.wmu);
        if ((rc = register_locked(host_w, type, k, n))) return rc;
    }
    return fail(QK_ERR_UNREGISTERED, "weight %p was unregistered during the call", host_w);
}

// Prefill GEMMs on Q5_K / Q6_K weights run on int8 MFMA planes
// (hip_matmul_planes), made once per weight on its first prefill: release
// the shared lock, pack under the exclusive one (synchronously, so no
// other stream sees half-written planes), and take the shared lock again.
bool planes_pay(int type) { return type == QK_TYPE_Q5_K || type == QK_TYPE_Q6_K; }

int acquire_planes(const void *host_w, int type, int64_t k, int64_t n, hipStream_t stream,
                   std::shared_lock<std::shared_mutex> &rl, Weight *out) {
    State &s = st();
    int rc;
    if (out->planes) return QK_OK;
    rl.unlock();
    {
        std::unique_lock<std::shared_mutex> wl(s.wmu);
        auto it = s.weights.find(host_w);
        if (it != s.weights.end() && !it->second.planes) {
            Weight &w = it->second;
            void *p = nullptr;
            HIP_OK(hipMalloc(&p, qk::gemm_planes_bytes(type, n, k)), "hipMalloc(planes)");
            hipError_t e = qk::launch_pack_planes(type, static_cast<const uint8_t *>(w.dev), n, k,
                                                  static_cast<uint8_t *>(p), stream);
            if (e == hipSuccess) e = hipStreamSynchronize(stream);
            if (e != hipSuccess) {
                (void)hipFree(p);
                return hip_fail(e, "pack planes");
            }
            w.planes = p;
        }
    }
    if ((rc = acquire_weight(host_w, type, k, n, rl, out))) return rc;
    if (!out->planes) return fail(QK_ERR_UNREGISTERED, "weight %p was re-registered during the call", host_w);
    return QK_OK;
}
}  // namespace

extern "C" {

int hip_qk_register_weight(const void *host_w, int type, int64_t k, int64_t n) {
    int rc = require_init();
    if (rc) return rc;
    if ((rc = check_weight_args(host_w, type, k, n))) return rc;
    if ((rc = ensure_device())) return rc;
    std::unique_lock<std::shared_mutex> wl(st().wmu);
    return register_locked(host_w, type, k, n);
}

int hip_qk_unregister_weight(const void *host_w) {
    State &s = st();
    int rc;
    if ((rc = require_init())) return rc;
    if ((rc = ensure_device())) return rc;
    std::unique_lock<std::shared_mutex> wl(s.wmu);
    auto it = s.weights.find(host_w);
    if (it == s.weights.end()) return fail(QK_ERR_UNREGISTERED, "weight %p is not registered", host_w);
    free_weight(it->second);
    s.weights.erase(it);
    return QK_OK;
}

int hip_qk_unregister_range(const void *base, size_t bytes) {
    State &s = st();
    if (!s.init || !base || bytes == 0) return 0;
    if (ensure_device()) return 0;
    std::unique_lock<std::shared_mutex> wl(s.wmu);
    const uintptr_t lo = reinterpret_cast<uintptr_t>(base), hi = lo + bytes;
    int count = 0;
    for (auto it = s.weights.begin(); it != s.weights.end();) {
        const uintptr_t a = reinterpret_cast<uintptr_t>(it->first), b = a + it->second.bytes;
        if (a < hi && lo < b) {
            free_weight(it->second);
            it = s.weights.erase(it);
            count++;
        } else {
            ++it;
        }
    }
    return count;
}

const void *hip_qk_device_weight(const void *host_w) {
    State &s = st();
    std::shared_lock<std::shared_mutex> rl(s.wmu);
    auto it = s.weights.find(host_w);
    return it == s.weights.end() ? nullptr : it->second.dev;
}

int hip_qk_matmul_host(const void *host_w, int type, int64_t out_f, int64_t k, const float *x,
                       int64_t n_tok, float *out) {
    int rc = require_init();
    if (rc) return rc;
    if (!x || !out || n_tok < 1) return fail(QK_ERR_ARG, "bad activation arguments");
    if ((rc = check_weight_args(host_w, type, k, out_f))) return rc;
    if (n_tok > gemm_max_m(type))
        return fail(QK_ERR_ARG, "n_tok=%lld tokens (1..%lld)", (long long)n_tok, (long long)gemm_max_m(type));
    Lane *l = nullptr;
    if ((rc = my_lane(&l))) return rc;
    std::shared_lock<std::shared_mutex> rl;
    Weight w;
    if ((rc = acquire_weight(host_w, type, k, out_f, rl, &w))) return rc;
    if (n_tok > 1 && planes_pay(type) && (rc = acquire_planes(host_w, type, k, out_f, l->stream, rl, &w))) return rc;
    const size_t xb = (size_t)(n_tok * k) * sizeof(float);
    const size_t qb = (size_t)(n_tok * act_bytes(type, k));
    const size_t yb = (size_t)(n_tok * out_f) * sizeof(float);
    if ((rc = grow(&l->dx, &l->dx_cap, xb)) || (rc = grow(&l->dxq, &l->dxq_cap, qb)) ||
        (rc = grow(&l->dy, &l->dy_cap, yb)) || (rc = grow_host(&l->hx, &l->hx_cap, xb)) ||
        (rc = grow_host(&l->hy, &l->hy_cap, yb)))
        return rc;
    // x through pinned memory: a decode row (<= 16 KB) is read by the
    // quantizer straight from host memory; a prefill chunk goes by DMA.
    std::memcpy(l->hx, x, xb);
    void *hx_dev = nullptr;
    HIP_OK(hipHostGetDevicePointer(&hx_dev, l->hx, 0), "hipHostGetDevicePointer");
    const float *dx = static_cast<const float *>(hx_dev);
    if (xb > 16384) {
        HIP_OK(hipMemcpyAsync(l->dx, l->hx, xb, hipMemcpyHostToDevice, l->stream), "hipMemcpyAsync(x)");
        dx = static_cast<const float *>(l->dx);
    }
    uint8_t *dxq = static_cast<uint8_t *>(l->dxq);
    // y likewise: a small output (decode rows, <= 64 KB) is written by the
    // kernel straight into pinned host memory; a larger one goes by DMA.
    float *dy = static_cast<float *>(l->dy);
    const bool y_direct = yb <= 65536;
    if (y_direct) {
        void *hy_dev = nullptr;
        HIP_OK(hipHostGetDevicePointer(&hy_dev, l->hy, 0), "hipHostGetDevicePointer");
        dy = static_cast<float *>(hy_dev);
    }
    // the same contract as the device layer, on the device copy
    if ((rc = check_mat(type, w.dev, out_f, k, dxq, dy))) return rc;
    const int fused = fused_of(st().tier.load());
    if (type == QK_TYPE_Q8_0) HIP_OK(qk::launch_quantize_q8_0(dx, n_tok * (k / QK8_0), dxq, l->stream), "quantize");
    else HIP_OK(qk::launch_quantize_q8k(dx, n_tok * (k / QK_K), dxq, l->stream), "quantize");
    if (n_tok == 1) {
        qk::GemvArgs a{};
        a.fused = fused;
        a.count = 1;
        a.d[0].type = type;
        a.d[0].n = out_f;
        a.d[0].k = k;
        a.d[0].w = static_cast<const uint8_t *>(w.dev);
        a.d[0].xq = dxq;
        a.d[0].y = dy;
        qk::gemv_plan(a.d[0]);
        HIP_OK(qk::launch_gemv(a, matvec_grid(type), l->stream), "gemv launch");
    } else if (planes_pay(type)) {
        HIP_OK(qk::launch_gemm_planes(type, static_cast<const uint8_t *>(w.planes), out_f, k, dxq, n_tok, dy, fused,
                                      l->stream),
               "gemm launch");
    } else {
        HIP_OK(qk::launch_gemm(type, static_cast<const uint8_t *>(w.dev), out_f, k, dxq, n_tok, dy, fused, l->stream),
               "gemm launch");
    }
    if (!y_direct)
        HIP_OK(hipMemcpyAsync(l->hy, dy, yb, hipMemcpyDeviceToHost, l->stream), "hipMemcpyAsync(out)");
    HIP_OK(hipStreamSynchronize(l->stream), "hipStreamSynchronize");
    std::memcpy(out, l->hy, yb);
    return QK_OK;
}

int hip_qk_lmhead_host(const void *host_w, int64_t n, int64_t k, const float *x, int topk,
                       float *logits, int32_t *argmax, int32_t *topk_idx, float *topk_val) {
    int rc = require_init();
    if (rc) return rc;
    if (!x) return fail(QK_ERR_ARG, "bad arguments");
    if ((rc = check_lmhead_outputs(n, topk, argmax, topk_idx, topk_val))) return rc;
    if ((rc = check_weight_args(host_w, QK_TYPE_Q6_K, k, n))) return rc;
    Lane *l = nullptr;
    if ((rc = my_lane(&l))) return rc;
    std::shared_lock<std::shared_mutex> rl;
    Weight w;
    if ((rc = acquire_weight(host_w, QK_TYPE_Q6_K, k, n, rl, &w))) return rc;
    const size_t xb = (size_t)k * sizeof(float);
    const size_t qb = (size_t)act_bytes(QK_TYPE_Q6_K, k);
    // dy: logits (n) | argmax (1) | topk idx (QK_TOPK_MAX) | topk val (QK_TOPK_MAX)
    const size_t yb = (size_t)(n + 1 + 2 * QK_TOPK_MAX) * sizeof(float) + 64;
    // the lane's stream finishes every call before returning, so its
    // scratch can be replaced freely
    if ((rc = grow(&l->dx, &l->dx_cap, xb)) || (rc = grow(&l->dxq, &l->dxq_cap, qb)) ||
        (rc = grow(&l->dy, &l->dy_cap, yb)) ||
        (rc = grow(&l->dsel, &l->dsel_cap, lmhead_scratch_bytes(n, topk, false))))
        return rc;
    HIP_OK(hipMemcpyAsync(l->dx, x, xb, hipMemcpyHostToDevice, l->stream), "hipMemcpyAsync(x)");
    HIP_OK(qk::launch_quantize_q8k(static_cast<const float *>(l->dx), k / QK_K, static_cast<uint8_t *>(l->dxq),
                                   l->stream),
           "quantize");
    float *dl = static_cast<float *>(l->dy);
    int32_t *dam = reinterpret_cast<int32_t *>(dl + n);
    int32_t *dti = dam + 1;
    float *dtv = reinterpret_cast<float *>(dti + QK_TOPK_MAX);
    if ((rc = lmhead_launch(w.dev, n, k, l->dxq, topk, dl, dam, dti, dtv, l->dsel, l->stream))) return rc;
    if (logits)
        HIP_OK(hipMemcpyAsync(logits, dl, (size_t)n * sizeof(float), hipMemcpyDeviceToHost, l->stream), "copy logits");
    HIP_OK(hipMemcpyAsync(argmax, dam, sizeof(int32_t), hipMemcpyDeviceToHost, l->stream), "copy argmax");
    if (topk > 0) {
        HIP_OK(hipMemcpyAsync(topk_idx, dti, (size_t)topk * sizeof(int32_t), hipMemcpyDeviceToHost, l->stream),
               "copy topk idx");
        HIP_OK(hipMemcpyAsync(topk_val, dtv, (size_t)topk * sizeof(float), hipMemcpyDeviceToHost, l->stream),
               "copy topk val");
    }
    HIP_OK(hipStreamSynchronize(l->stream), "hipStreamSynchronize");
    return QK_OK;
}

int hip_qk_deltanet_host(int n, int k_hd, int v_hd, const float *q, const float *k, const float *v,
                         const float *g_log, const float *beta, float *state, float *out) {
    int rc = require_host_expf("hip_qk_deltanet_host");
    if (rc) return rc;
    rc = require_init();
    if (rc) return rc;
    if (!q || !k || !v || !g_log || !beta || !state || !out) return fail(QK_ERR_ARG, "null pointer");
    if (n < 1 || n > 64 || k_hd < 1 || v_hd < 1 || k_hd > QK_DELTANET_MAX_HD || v_hd > QK_DELTANET_MAX_HD)
        return fail(QK_ERR_ARG, "bad chunk n=%d k_hd=%d v_hd=%d (n 1..64, head dims 1..%d)", n, k_hd, v_hd,
                    QK_DELTANET_MAX_HD);
    return deltanet_host(n, 1, k_hd, v_hd, q, k, v, g_log, beta, state, out);
}

int hip_qk_deltanet_layer_host(int64_t n_tok, int n_heads, int k_hd, int v_hd, const float *q, const float *k,
                               const float *v, const float *g_log, const float *beta, float *state, float *out) {
    int rc = require_host_expf("hip_qk_deltanet_layer_host");
    if (rc) return rc;
    rc = require_init();
    if (rc) return rc;
    if (!q || !k || !v || !g_log || !beta || !state || !out) return fail(QK_ERR_ARG, "null pointer");
    if (n_tok < 1 || n_tok > 0x7fffffffLL || n_heads < 1 || n_heads > 1024 || k_hd < 1 || v_hd < 1 ||
        k_hd > QK_DELTANET_MAX_HD || v_hd > QK_DELTANET_MAX_HD)
        return fail(QK_ERR_ARG, "bad shape n_tok=%lld heads=%d k_hd=%d v_hd=%d (head dims 1..%d)", (long long)n_tok,
                    n_heads, k_hd, v_hd, QK_DELTANET_MAX_HD);
    // q, k, v, g, beta, state and out staged at once
    const double bytes = 4.0 * (double)n_tok * n_heads * (2.0 * k_hd + 2.0 * v_hd + 2.0) +
                         4.0 * (double)n_heads * k_hd * v_hd;
    if (bytes > QK_DELTANET_HOST_MAX_BYTES)
        return fail(QK_ERR_ARG, "layer of %.0f bytes exceeds QK_DELTANET_HOST_MAX_BYTES; split the tokens", bytes);
    return deltanet_host(n_tok, n_heads, k_hd, v_hd, q, k, v, g_log, beta, state, out);
}

}  // extern "C"
