// Model-level C ABI: device context, HybridMambaModel weights and forward/prefill/decode,
// recurrent state, checkpoint load/export and greedy generation.
//
// Mirrors what the reference's session layer calls on MambaCode.js (see include/ssm_hip.h):
// new HybridMambaModel (src/session/session.ts:359), model.forward (src/session/streaming.ts:
// 31-35), model.generate (session.ts:421-425), loadWeights / exportWeights (session.ts:394,518,
// 575). The architecture matches the canonical Mamba / Mamba-2 blocks:
//   embedding -> n_layers x [x += mixer(RMSNorm(x))] -> RMSNorm -> tied LM head
//   mamba1 mixer: in_proj -> (x, z); x = SiLU(conv(x)); (dt, B, C) = x_proj(x);
//                 dt = dt_proj(dt); y = scan(x, dt, A, B, C, D, z, softplus(dt + bias)); out_proj
//   mamba2 mixer: in_proj -> (z, xBC, dt); xBC = SiLU(conv(xBC)); y = SSD(x, dt, A, B, C, D);
//                 y = RMSNorm_grouped(y * SiLU(z)); out_proj
// Projections are rocBLAS SGEMMs on the context stream; the residual add is folded into the
// out_proj GEMM (beta = 1).
#include <hipblaslt/hipblaslt.h>
#include <rocblas/rocblas.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <map>
#include <mutex>
#include <tuple>
#include <string>
#include <vector>

#include "common.hpp"
#include "glue.hpp"
#include "ssd.hpp"
#include "ssmw.hpp"

// ------------------------------------------------------------------ errors
namespace ssm {

static thread_local std::string g_err;

void set_error(const char* fmt, ...) {
    char buf[1024];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_err = buf;
}

ssm_status fail(ssm_status code, const char* fmt, ...) {
    char buf[1024];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_err = buf;
    return code;
}

ssm_status from_hip(hipError_t e, const char* what) {
    ssm_status code = SSM_ERR_HIP;
    if (e == hipErrorOutOfMemory) code = SSM_ERR_OUT_OF_MEMORY;
    if (e == hipErrorNoDevice || e == hipErrorInvalidDevice) code = SSM_ERR_GPU_UNAVAILABLE;
    return fail(code, "%s: %s", what, hipGetErrorString(e));
}

// Fault injection for tests of the error contract (session.ts:262-270,393-401): a failure the
// library reports as if HIP had returned it. "nodevice": ssm_ctx_create finds no device;
// "alloc": every device allocation of the library fails (out of memory); "launch": every
// launch check reports a failed launch after the (normally running) kernel was queued.
// The kind lives in an atomic: ssm_set_fault_injection sets it (and pins it against the
// environment until it is called with NULL); otherwise each ssm_ctx_create latches the
// environment variable SSM_HIP_FAULT into it. Nothing reads the environment per launch or
// allocation (getenv is not safe against a concurrent setenv on another thread).
enum FaultKind { kFaultNone = 0, kFaultNoDevice, kFaultAlloc, kFaultLaunch, kFaultUnknown };
std::atomic<int> g_fault{kFaultNone};
std::atomic<bool> g_fault_pinned{false};

int parse_fault(const char* f) {
    if (!f || !*f) return kFaultNone;
    if (std::strcmp(f, "nodevice") == 0) return kFaultNoDevice;
    if (std::strcmp(f, "alloc") == 0) return kFaultAlloc;
    if (std::strcmp(f, "launch") == 0) return kFaultLaunch;
    return kFaultUnknown;
}

void latch_fault_env() {
    if (!g_fault_pinned.load(std::memory_order_acquire))
        g_fault.store(parse_fault(std::getenv("SSM_HIP_FAULT")), std::memory_order_release);
}

bool fault(int kind) { return g_fault.load(std::memory_order_relaxed) == kind; }

hipError_t dev_malloc(void** p, size_t bytes) {
    if (fault(kFaultAlloc)) {
        *p = nullptr;
        return hipErrorOutOfMemory;
    }
    return hipMalloc(p, bytes);
}

ssm_status check_launch(const char* what) {
    hipError_t e = hipGetLastError();
    if (e == hipSuccess && fault(kFaultLaunch))
        return fail(SSM_ERR_HIP, "%s: launch failure (injected fault: launch)", what);
    return e == hipSuccess ? SSM_OK : from_hip(e, what);
}

}  // namespace ssm

#define SSM_TRY(expr)                       \
    do {                                    \
        ssm_status _s = (expr);             \
        if (_s != SSM_OK) return _s;        \
    } while (0)

extern "C" const char* ssm_last_error(void) { return ssm::g_err.c_str(); }

extern "C" const char* ssm_status_name(ssm_status s) {
    switch (s) {
        case SSM_OK: return "OK";
        case SSM_ERR_GPU_UNAVAILABLE: return "GPU_UNAVAILABLE";
        case SSM_ERR_CHECKPOINT_INVALID: return "CHECKPOINT_INVALID";
        case SSM_ERR_DESTROYED: return "SESSION_DESTROYED";
        default: return "UNKNOWN";
    }
}

extern "C" int ssm_abi_version(void) { return 1; }

extern "C" ssm_status ssm_set_fault_injection(const char* kind) {
    if (!kind) {
        ssm::g_fault_pinned.store(false, std::memory_order_release);
        ssm::g_fault.store(ssm::kFaultNone, std::memory_order_release);
        return SSM_OK;
    }
    const int k = ssm::parse_fault(kind);
    if (k == ssm::kFaultUnknown)
        return ssm::fail(SSM_ERR_INVALID_ARG, "ssm_set_fault_injection: unknown kind '%s'", kind);
    ssm::g_fault.store(k, std::memory_order_release);
    ssm::g_fault_pinned.store(true, std::memory_order_release);
    return SSM_OK;
}

// ------------------------------------------------------------------ context
constexpr size_t kLtWorkspace = 32u << 20;   // hipBLASLt workspace per context

struct ssm_ctx {
    int device = 0;
    hipStream_t own = nullptr;
    hipStream_t stream = nullptr;
    rocblas_handle blas = nullptr;
    // hipBLASLt for the projection GEMMs with K >= 128 (its fp32 kernels measured 5-25% faster
    // than rocBLAS's on this chip for the model's shapes); one plan (descriptor, layouts and
    // the heuristic's first algorithm) per shape
    hipblasLtHandle_t lt = nullptr;
    void* lt_ws = nullptr;
    struct LtPlan {
        bool ok = false;
        hipblasLtMatmulDesc_t desc = nullptr;
        hipblasLtMatrixLayout_t la = nullptr, lb = nullptr, lc = nullptr;
        hipblasLtMatmulAlgo_t algo{};
    };
    // key (M, N, K, ldx, ldy, operand type): HIP_R_32F, or HIP_R_16BF operands with fp32
    // accumulation and output (the bf16-input layer)
    std::map<std::tuple<int, int, int, long, long, int>, LtPlan> lt_plans;
    bool destroyed = false;
    // Held by every entry point that uses the context (its stream, BLAS handles, plan cache,
    // profiler record, and the workspaces and graphs of models and states made on it) for the
    // whole call, including host synchronisation and graph capture. Calls from several
    // threads on one device (the Node-API addon runs each Promise on a pool thread) are
    // therefore serialised, a capture never records another caller's launches, and
    // ssm_ctx_destroy waits for the call in flight. Recursive: entry points call each other.
    std::recursive_mutex mu;
    char arch[64] = {0};
    int cus = 0;
    size_t mem = 0;
    // opt-in stage profiler: (stage, start, stop) event pairs on the context stream
    bool prof = false;
    struct Mark { const char* name; hipEvent_t a, b; };
    std::vector<Mark> marks;
};

namespace {

// Records a start event on construction and a stop event on destruction when profiling.
struct Stage {
    ssm_ctx* c;
    size_t idx = (size_t)-1;
    Stage(ssm_ctx* ctx, const char* name) : c(ctx) {
        if (!c->prof) return;
        ssm_ctx::Mark mk{name, nullptr, nullptr};
        if (hipEventCreate(&mk.a) != hipSuccess || hipEventCreate(&mk.b) != hipSuccess) return;
        hipEventRecord(mk.a, c->stream);
        c->marks.push_back(mk);
        idx = c->marks.size() - 1;
    }
    ~Stage() {
        if (idx != (size_t)-1) hipEventRecord(c->marks[idx].b, c->stream);
    }
};

ssm_status blas_status(rocblas_status s, const char* what) {
    if (s == rocblas_status_success) return SSM_OK;
    return ssm::fail(SSM_ERR_HIP, "%s: rocBLAS status %d", what, (int)s);
}

using CtxLock = std::unique_lock<std::recursive_mutex>;

// Checks run with the context lock held.
ssm_status ctx_live(ssm_ctx* c) {
    if (c->destroyed) return ssm::fail(SSM_ERR_DESTROYED, "context has been destroyed");
    SSM_HIP_TRY(hipSetDevice(c->device));
    return SSM_OK;
}

// Takes the context lock into `lk` (kept until the caller returns), then checks the context.
ssm_status ctx_enter(ssm_ctx* c, CtxLock& lk) {
    if (!c) return ssm::fail(SSM_ERR_INVALID_ARG, "null context");
    lk = CtxLock(c->mu);
    return ctx_live(c);
}

// The hipBLASLt plan of a shape: Y^T (Nout x M, column-major, ld ldy) = op(A) B with A = W
// as a K x Nout column-major matrix (transposed) and B = X^T as K x M (ld ldx), fp32 compute.
// The heuristic's first algorithm is taken (no timing runs), so the choice, and the bits of
// the result, are the same in every process. ok = false leaves the shape to rocBLAS.
ssm_ctx::LtPlan& lt_plan(ssm_ctx* c, int M, int Nout, int K, long ldx, long ldy,
                        hipDataType ab = HIP_R_32F) {
    auto& p = c->lt_plans[std::make_tuple(M, Nout, K, ldx, ldy, (int)ab)];
    if (p.desc) return p;
    const hipblasOperation_t ta = HIPBLAS_OP_T, tb = HIPBLAS_OP_N;
    bool ok = hipblasLtMatmulDescCreate(&p.desc, HIPBLAS_COMPUTE_32F, HIP_R_32F) == HIPBLAS_STATUS_SUCCESS &&
              hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSA, &ta, sizeof ta) == HIPBLAS_STATUS_SUCCESS &&
              hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSB, &tb, sizeof tb) == HIPBLAS_STATUS_SUCCESS &&
              hipblasLtMatrixLayoutCreate(&p.la, ab, K, Nout, K) == HIPBLAS_STATUS_SUCCESS &&
              hipblasLtMatrixLayoutCreate(&p.lb, ab, K, M, ldx) == HIPBLAS_STATUS_SUCCESS &&
              hipblasLtMatrixLayoutCreate(&p.lc, HIP_R_32F, Nout, M, ldy) == HIPBLAS_STATUS_SUCCESS;
    if (ok) {
        hipblasLtMatmulPreference_t pref = nullptr;
        size_t wsb = kLtWorkspace;
        hipblasLtMatmulHeuristicResult_t res{};
        int n = 0;
        ok = hipblasLtMatmulPreferenceCreate(&pref) == HIPBLAS_STATUS_SUCCESS &&
             hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES,
                                                   &wsb, sizeof wsb) == HIPBLAS_STATUS_SUCCESS &&
             hipblasLtMatmulAlgoGetHeuristic(c->lt, p.desc, p.la, p.lb, p.lc, p.lc, pref, 1, &res,
                                             &n) == HIPBLAS_STATUS_SUCCESS &&
             n > 0;
        if (pref) hipblasLtMatmulPreferenceDestroy(pref);
        if (ok) p.algo = res.algo;
    }
    p.ok = ok;
    return p;
}

// Y (M, Nout) [ld ldy] = X (M, K) [ld ldx] * W^T, W (Nout, K) row-major; Y = beta*Y + ...
// Products of M >= kOwnGemmRows rows run the fp32 matrix-core kernel of gemm.hip (split over
// K when its tiles leave CUs idle and a workspace is given); the prefill of up to
// kFewRows tokens runs the row kernel of rowgemm.hip (proj_rows); the rest (prompts of 65 to
// 255 tokens, the one-token fallbacks) go to hipBLASLt for K >= 128 (below that rocBLAS
// measured faster) and rocBLAS for the rest and any shape hipBLASLt has no algorithm for.
// SSM_GEMM=lib sends every product to the libraries, SSM_GEMM=rocblas everything to rocBLAS.
constexpr int kOwnGemmRows = 256;
constexpr int kFewRows = 64;
bool lib_only() {
    static const bool v = [] {
        const char* e = std::getenv("SSM_GEMM");
        return e && (std::strcmp(e, "lib") == 0 || std::strcmp(e, "rocblas") == 0);
    }();
    return v;
}
bool own_kernels(int M) { return !lib_only() && M >= kOwnGemmRows; }
bool few_rows(int M) { return !lib_only() && M >= 1 && M <= kFewRows; }
// part / part_n: the own kernel's split-K workspace (gemm.hip; null runs unsplit).
ssm_status gemm(ssm_ctx* c, int M, int Nout, int K, const float* X, long ldx, const float* W,
                float* Y, long ldy, float beta, float* part = nullptr, size_t part_n = 0) {
    if (M == 0 || Nout == 0) return SSM_OK;
    const float one = 1.f;
    static const bool rb_only = [] {
        const char* e = std::getenv("SSM_GEMM");
        return e && std::strcmp(e, "rocblas") == 0;
    }();
    if (own_kernels(M) && ssm::gemm_ok(M, Nout, K, ldx, K, ldy) &&
        (((uintptr_t)X | (uintptr_t)W) & 15) == 0)
        return ssm::launch_gemm(X, ldx, W, K, nullptr, Y, ldy, M, Nout, K, beta, c->stream,
                                nullptr, 0, 0.f, 0.f, 0x7fffffff, part, part_n);
    if (c->lt && K >= 128 && !rb_only) {
        auto& p = lt_plan(c, M, Nout, K, ldx, ldy);
        if (p.ok) {
            const hipblasStatus_t s = hipblasLtMatmul(c->lt, p.desc, &one, W, p.la, X, p.lb, &beta,
                                                      Y, p.lc, Y, p.lc, &p.algo, c->lt_ws,
                                                      kLtWorkspace, c->stream);
            if (s != HIPBLAS_STATUS_SUCCESS)
                return ssm::fail(SSM_ERR_HIP, "hipblasLtMatmul: status %d", (int)s);
            return SSM_OK;
        }
    }
    return blas_status(rocblas_sgemm(c->blas, rocblas_operation_transpose, rocblas_operation_none,
                                     Nout, M, K, &one, W, K, X, (rocblas_int)ldx, &beta, Y,
                                     (rocblas_int)ldy),
                       "sgemm");
}

// Y (M, Nout) fp32 [ld ldy] = beta*Y + X W^T with bf16 X (M, K) [ld ldx] and W (Nout, K)
// row-major, fp32 accumulation: a plain library GEMM (hipBLASLt).
ssm_status gemm_bf16(ssm_ctx* c, int M, int Nout, int K, const __bf16* X, long ldx,
                     const __bf16* W, float* Y, long ldy, float beta) {
    if (M == 0 || Nout == 0) return SSM_OK;
    if (!c->lt) return ssm::fail(SSM_ERR_HIP, "bf16 GEMM: hipBLASLt unavailable");
    auto& p = lt_plan(c, M, Nout, K, ldx, ldy, HIP_R_16BF);
    if (!p.ok) return ssm::fail(SSM_ERR_HIP, "bf16 GEMM: no hipBLASLt algorithm for %d x %d x %d",
                                M, Nout, K);
    const float one = 1.f;
    const hipblasStatus_t s = hipblasLtMatmul(c->lt, p.desc, &one, W, p.la, X, p.lb, &beta, Y,
                                              p.lc, Y, p.lc, &p.algo, c->lt_ws, kLtWorkspace,
                                              c->stream);
    if (s != HIPBLAS_STATUS_SUCCESS) return ssm::fail(SSM_ERR_HIP, "hipblasLtMatmul (bf16): status %d", (int)s);
    return SSM_OK;
}

}  // namespace

extern "C" ssm_status ssm_ctx_create(int device_ordinal, ssm_ctx** out) {
    if (!out) return ssm::fail(SSM_ERR_INVALID_ARG, "ssm_ctx_create: null out");
    *out = nullptr;
    ssm::latch_fault_env();
    if (ssm::fault(ssm::kFaultNoDevice))
        return ssm::fail(SSM_ERR_GPU_UNAVAILABLE, "no HIP device (injected fault: nodevice)");
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess || n == 0)
        return ssm::fail(SSM_ERR_GPU_UNAVAILABLE, "no HIP device available (%s)",
                         e != hipSuccess ? hipGetErrorString(e) : "device count 0");
    if (device_ordinal < 0 || device_ordinal >= n)
        return ssm::fail(SSM_ERR_GPU_UNAVAILABLE, "device %d out of range (%d devices)",
                         device_ordinal, n);
    ssm_ctx* c = new ssm_ctx();
    c->device = device_ordinal;
    hipDeviceProp_t prop;
    if ((e = hipSetDevice(device_ordinal)) != hipSuccess ||
        (e = hipGetDeviceProperties(&prop, device_ordinal)) != hipSuccess ||
        (e = hipStreamCreateWithFlags(&c->own, hipStreamNonBlocking)) != hipSuccess) {
        delete c;
        return ssm::from_hip(e, "ssm_ctx_create");
    }
    // the allocation-free sampler's scratch address on this device, resolved here so that a
    // caller's first ssm_sample_noalloc (possibly under graph capture) makes no runtime lookup
    {
        void* scratch = nullptr;
        const ssm_status sr = ssm::sample_scratch(&scratch);
        if (sr != SSM_OK) {
            hipStreamDestroy(c->own);
            delete c;
            return sr;
        }
    }
    std::snprintf(c->arch, sizeof c->arch, "%s", prop.gcnArchName);
    c->cus = prop.multiProcessorCount;
    c->mem = prop.totalGlobalMem;
    c->stream = c->own;
    if (rocblas_create_handle(&c->blas) != rocblas_status_success ||
        rocblas_set_stream(c->blas, c->stream) != rocblas_status_success) {
        hipStreamDestroy(c->own);
        delete c;
        return ssm::fail(SSM_ERR_GPU_UNAVAILABLE, "rocBLAS handle creation failed");
    }
    // without hipBLASLt (or its workspace) every GEMM goes to rocBLAS
    if (hipblasLtCreate(&c->lt) != HIPBLAS_STATUS_SUCCESS) c->lt = nullptr;
    if (c->lt && ssm::dev_malloc(&c->lt_ws, kLtWorkspace) != hipSuccess) {
        hipblasLtDestroy(c->lt);
        c->lt = nullptr;
        c->lt_ws = nullptr;
    }
    *out = c;
    return SSM_OK;
}

extern "C" ssm_status ssm_ctx_destroy(ssm_ctx* c) {
    if (!c) return SSM_OK;
    CtxLock lk(c->mu);   // waits for a call in flight on another thread
    if (!c->destroyed) {
        hipSetDevice(c->device);
        hipStreamSynchronize(c->stream);
        rocblas_destroy_handle(c->blas);
        for (auto& kv : c->lt_plans) {
            if (kv.second.desc) hipblasLtMatmulDescDestroy(kv.second.desc);
            if (kv.second.la) hipblasLtMatrixLayoutDestroy(kv.second.la);
            if (kv.second.lb) hipblasLtMatrixLayoutDestroy(kv.second.lb);
            if (kv.second.lc) hipblasLtMatrixLayoutDestroy(kv.second.lc);
        }
        c->lt_plans.clear();
        if (c->lt) hipblasLtDestroy(c->lt);
        hipFree(c->lt_ws);
        hipStreamDestroy(c->own);
        c->destroyed = true;
    }
    // The struct is kept (not freed) so that models still holding it see SESSION_DESTROYED.
    return SSM_OK;
}

extern "C" ssm_status ssm_ctx_set_stream(ssm_ctx* c, void* stream) {
    CtxLock lk;
    SSM_TRY(ctx_enter(c, lk));
    c->stream = stream ? (hipStream_t)stream : c->own;
    return blas_status(rocblas_set_stream(c->blas, c->stream), "rocblas_set_stream");
}

extern "C" void* ssm_ctx_stream(ssm_ctx* c) { return c ? (void*)c->stream : nullptr; }

extern "C" ssm_status ssm_ctx_profile(ssm_ctx* c, int enable) {
    CtxLock lk;
    SSM_TRY(ctx_enter(c, lk));
    c->prof = enable != 0;
    return SSM_OK;
}

extern "C" ssm_status ssm_ctx_profile_report(ssm_ctx* c, char* buf, size_t cap) {
    CtxLock lk;
    SSM_TRY(ctx_enter(c, lk));
    SSM_HIP_TRY(hipStreamSynchronize(c->stream));
    std::vector<std::string> names;
    std::vector<double> tot;
    std::vector<long> cnt;
    for (const ssm_ctx::Mark& mk : c->marks) {
        float ms = 0.f;
        if (hipEventElapsedTime(&ms, mk.a, mk.b) != hipSuccess) ms = 0.f;
        size_t i = 0;
        while (i < names.size() && names[i] != mk.name) ++i;
        if (i == names.size()) { names.push_back(mk.name); tot.push_back(0.0); cnt.push_back(0); }
        tot[i] += ms;
        cnt[i] += 1;
        hipEventDestroy(mk.a);
        hipEventDestroy(mk.b);
    }
    c->marks.clear();
    std::string out;
    char line[256];
    for (size_t i = 0; i < names.size(); ++i) {
        std::snprintf(line, sizeof line, "%s %ld %.6f\n", names[i].c_str(), cnt[i], tot[i]);
        out += line;
    }
    if (buf && cap) std::snprintf(buf, cap, "%s", out.c_str());
    return SSM_OK;
}

extern "C" ssm_status ssm_ctx_synchronize(ssm_ctx* c) {
    CtxLock lk;
    SSM_TRY(ctx_enter(c, lk));
    SSM_HIP_TRY(hipStreamSynchronize(c->stream));
    return SSM_OK;
}

extern "C" ssm_status ssm_ctx_info(ssm_ctx* c, char* arch, int arch_len, int* cus,
                                   size_t* mem) {
    CtxLock lk;
    SSM_TRY(ctx_enter(c, lk));
    if (arch && arch_len > 0) std::snprintf(arch, arch_len, "%s", c->arch);
    if (cus) *cus = c->cus;
    if (mem) *mem = c->mem;
    return SSM_OK;
}

extern "C" ssm_status ssm_malloc(ssm_ctx* c, size_t bytes, void** dptr) {
    CtxLock lk;
    SSM_TRY(ctx_enter(c, lk));
    SSM_REQUIRE(dptr, "ssm_malloc: null out");
    SSM_HIP_TRY(ssm::dev_malloc(dptr, bytes ? bytes : 1));
    return SSM_OK;
}
extern "C" ssm_status ssm_free(ssm_ctx* c, void* p) {
    CtxLock lk;
    SSM_TRY(ctx_enter(c, lk));
    SSM_HIP_TRY(hipStreamSynchronize(c->stream));
    SSM_HIP_TRY(hipFree(p));
    return SSM_OK;
}
extern "C" ssm_status ssm_memcpy_h2d(ssm_ctx* c, void* dst, const void* src, size_t n) {
    CtxLock lk;
    SSM_TRY(ctx_enter(c, lk));
    SSM_HIP_TRY(hipMemcpyAsync(dst, src, n, hipMemcpyHostToDevice, c->stream));
    SSM_HIP_TRY(hipStreamSynchronize(c->stream));
    return SSM_OK;
}
extern "C" ssm_status ssm_memcpy_d2h(ssm_ctx* c, void* dst, const void* src, size_t n) {
    CtxLock lk;
    SSM_TRY(ctx_enter(c, lk));
    SSM_HIP_TRY(hipMemcpyAsync(dst, src, n, hipMemcpyDeviceToHost, c->stream));
    SSM_HIP_TRY(hipStreamSynchronize(c->stream));
    return SSM_OK;
}

// ------------------------------------------------------------------ model
namespace {

struct LayerW {
    int type = 0;
    // offsets (floats) into the weight buffer; -1 when absent for the layer type
    long norm = -1, in_proj = -1, conv_w = -1, conv_b = -1, x_proj = -1, dt_w = -1, dt_b = -1,
         A_log = -1, Dsk = -1, gnorm = -1, out_proj = -1;
    long A = -1;  // offset into the A buffer (-exp(A_log))
};

struct Dims {
    int V, d, nl, N, K, expand, H, G, R, chunk, mimo, eos;
    float eps;
    int D, P, cd, nin;
};

}  // namespace

struct ssm_model {
    ssm_ctx* ctx = nullptr;
    Dims dm{};
    std::vector<int> types;
    std::vector<LayerW> layers;
    long emb = 0, norm_f = 0;
    size_t nfloats = 0, nA = 0;
    float* w = nullptr;      // weights in checkpoint payload order
    float* Ab = nullptr;     // A = -exp(A_log), per layer
    // workspace, grown on demand
    char* ws = nullptr;
    size_t ws_bytes = 0;
    // few-row projection split-K workspace (partial products), grown on demand
    char* rg = nullptr;
    size_t rg_bytes = 0;
    // in_proj / out_proj weights of the layers with a fused one-token step, in the step
    // projection's fragment order (stepproj.hip); built at the first such step and rebuilt
    // whenever the weights change
    float* wp = nullptr;
    std::vector<long> wp_in, wp_out;   // float offsets into wp per layer (-1: not packed)
    std::vector<long> wp_x, wp_dt;     // Mamba-1 layers: x_proj and dt_proj
    std::vector<long> wp_xt;           // Mamba-1 layers: x_proj transposed, (D, R + 2N)
    long wp_emb = -1;                  // the tied embedding for the one-token LM head
    // bf16 copies of the Mamba-2 layers' in_proj and out_proj for the bf16-input layer, built
    // at its first call and rebuilt whenever the weights change
    __bf16* wb = nullptr;
    std::vector<long> wb_in, wb_out;   // element offsets into wb per layer (-1: none)
    int* d_flag = nullptr;   // out-of-range token id flag
    uint32_t* d_ids = nullptr;
    size_t ids_cap = 0;
    bool destroyed = false;
};

struct ssm_state {
    ssm_model* m = nullptr;
    int B = 0;
    float* buf = nullptr;
    size_t floats = 0;
    std::vector<float*> ssm, conv;
    std::vector<size_t> ssm_n, conv_n;
    uint32_t* d_tok = nullptr;   // (B) ids for device decode steps
    uint32_t* d_gen = nullptr;   // generation ids ring
    size_t gen_cap = 0;
    float* d_logits = nullptr;   // (B, V)
    uint32_t* d_ping = nullptr;  // (2, B) ids of generation steps
    double* d_u = nullptr;       // (n_new, B) uniform draws of sampled generation
    size_t u_cap = 0;
    void* d_sws = nullptr;       // sampler workspace (ssm_sample_workspace(B, V) bytes)
    // Captured one-token steps: a step's kernels depend only on these pointers (the model's
    // weights and workspaces, this state's buffers, the ids / logits / argmax arguments), so a
    // step repeated with the same ones replays a HIP graph instead of launching ~5 kernels per
    // layer one by one.
    struct StepGraph {
        const uint32_t* ids;
        float* logits;
        uint32_t* argmax;
        const char* ws;
        const char* rg;
        hipGraphExec_t exec;
        uint64_t used;
    };
    std::vector<StepGraph> graphs;
    uint64_t graph_clock = 0;
    bool destroyed = false;
};

namespace {

// Model and state structs outlive their destroy calls (their flags answer later calls with
// SESSION_DESTROYED), so m->ctx and s->m stay readable; the flags are read under the lock.
ssm_status model_enter(ssm_model* m, CtxLock& lk) {
    if (!m) return ssm::fail(SSM_ERR_INVALID_ARG, "null model");
    lk = CtxLock(m->ctx->mu);
    if (m->destroyed) return ssm::fail(SSM_ERR_DESTROYED, "model has been destroyed");
    return ctx_live(m->ctx);
}

ssm_status state_enter(ssm_state* s, CtxLock& lk) {
    if (!s) return ssm::fail(SSM_ERR_INVALID_ARG, "null state");
    lk = CtxLock(s->m->ctx->mu);
    if (s->destroyed) return ssm::fail(SSM_ERR_DESTROYED, "state has been destroyed");
    if (s->m->destroyed) return ssm::fail(SSM_ERR_DESTROYED, "model has been destroyed");
    return ctx_live(s->m->ctx);
}

void build_layout(ssm_model* m) {
    const Dims& d = m->dm;
    long off = 0, aoff = 0;
    m->emb = off; off += (long)d.V * d.d;
    m->layers.assign(d.nl, LayerW());
    for (int l = 0; l < d.nl; ++l) {
        LayerW& L = m->layers[l];
        L.type = m->types[l];
        L.norm = off; off += d.d;
        if (L.type == SSM_LAYER_MAMBA1) {
            L.in_proj = off; off += 2L * d.D * d.d;
            L.conv_w = off; off += (long)d.D * d.K;
            L.conv_b = off; off += d.D;
            L.x_proj = off; off += (long)(d.R + 2 * d.N) * d.D;
            L.dt_w = off; off += (long)d.D * d.R;
            L.dt_b = off; off += d.D;
            L.A_log = off; off += (long)d.D * d.N;
            L.Dsk = off; off += d.D;
            L.out_proj = off; off += (long)d.d * d.D;
            L.A = aoff; aoff += (long)d.D * d.N;
        } else {
            L.in_proj = off; off += (long)d.nin * d.d;
            L.conv_w = off; off += (long)d.cd * d.K;
            L.conv_b = off; off += d.cd;
            L.dt_b = off; off += d.H;
            L.A_log = off; off += d.H;
            L.Dsk = off; off += d.H;
            L.gnorm = off; off += d.D;
            L.out_proj = off; off += (long)d.d * d.D;
            L.A = aoff; aoff += d.H;
        }
    }
    m->norm_f = off; off += d.d;
    m->nfloats = (size_t)off;
    m->nA = (size_t)aoff;
}

ssm_status pack_weights(ssm_model* m);

// bf16 (round to nearest even) copies of the Mamba-2 layers' in_proj and out_proj.
ssm_status build_wb(ssm_model* m) {
    const Dims& d = m->dm;
    hipStream_t st = m->ctx->stream;
    if (!m->wb) {
        m->wb_in.assign(d.nl, -1);
        m->wb_out.assign(d.nl, -1);
        long off = 0;
        for (int l = 0; l < d.nl; ++l) {
            if (m->types[l] != SSM_LAYER_MAMBA2) continue;
            m->wb_in[l] = off; off += ((long)d.nin * d.d + 127) / 128 * 128;
            m->wb_out[l] = off; off += ((long)d.d * d.D + 127) / 128 * 128;
        }
        if (off == 0) return SSM_OK;
        SSM_HIP_TRY(ssm::dev_malloc((void**)&m->wb, (size_t)off * sizeof(__bf16)));
    }
    for (int l = 0; l < d.nl; ++l) {
        if (m->wb_in[l] < 0) continue;
        const LayerW& Ly = m->layers[l];
        SSM_TRY(ssm::launch_cast_bf16(m->w + Ly.in_proj, d.d, m->wb + m->wb_in[l], d.d, d.nin,
                                      d.d, st));
        SSM_TRY(ssm::launch_cast_bf16(m->w + Ly.out_proj, d.D, m->wb + m->wb_out[l], d.D, d.d,
                                      d.D, st));
    }
    return SSM_OK;
}

// Everything derived from the weights: A = -exp(A_log) and, once built, the packed copies.
ssm_status refresh_A(ssm_model* m) {
    hipStream_t st = m->ctx->stream;
    for (const LayerW& L : m->layers) {
        const long n = L.type == SSM_LAYER_MAMBA1 ? (long)m->dm.D * m->dm.N : m->dm.H;
        SSM_TRY(ssm::launch_neg_exp(m->w + L.A_log, m->Ab + L.A, n, st));
    }
    if (m->wb) SSM_TRY(build_wb(m));
    return m->wp ? pack_weights(m) : SSM_OK;
}

ssm_status random_init(ssm_model* m, uint64_t seed) {
    const Dims& d = m->dm;
    hipStream_t st = m->ctx->stream;
    uint64_t tid = 0;
    auto I = [&](long off, long n, int kind, float a0, float a1, int row = 1) {
        return ssm::launch_init(m->w + off, n, kind, a0, a1, seed, tid++, row, st);
    };
    const float kb = 1.f / std::sqrt((float)d.K);
    SSM_TRY(I(m->emb, (long)d.V * d.d, SSM_INIT_NORMAL, 0.02f, 0.f));
    for (const LayerW& L : m->layers) {
        SSM_TRY(I(L.norm, d.d, SSM_INIT_CONST, 1.f, 0.f));
        if (L.type == SSM_LAYER_MAMBA1) {
            SSM_TRY(I(L.in_proj, 2L * d.D * d.d, SSM_INIT_NORMAL, 0.02f, 0.f));
            SSM_TRY(I(L.conv_w, (long)d.D * d.K, SSM_INIT_UNIFORM, -kb, kb));
            SSM_TRY(I(L.conv_b, d.D, SSM_INIT_UNIFORM, -kb, kb));
            SSM_TRY(I(L.x_proj, (long)(d.R + 2 * d.N) * d.D, SSM_INIT_NORMAL, 0.02f, 0.f));
            const float ds = 1.f / std::sqrt((float)d.R);
            SSM_TRY(I(L.dt_w, (long)d.D * d.R, SSM_INIT_UNIFORM, -ds, ds));
            SSM_TRY(I(L.dt_b, d.D, SSM_INIT_DT_BIAS, 1e-3f, 1e-1f));
            SSM_TRY(I(L.A_log, (long)d.D * d.N, SSM_INIT_ARANGE_LOG, 0.f, 0.f, d.N));
            SSM_TRY(I(L.Dsk, d.D, SSM_INIT_CONST, 1.f, 0.f));
            SSM_TRY(I(L.out_proj, (long)d.d * d.D, SSM_INIT_NORMAL, 0.02f, 0.f));
        } else {
            SSM_TRY(I(L.in_proj, (long)d.nin * d.d, SSM_INIT_NORMAL, 0.02f, 0.f));
            SSM_TRY(I(L.conv_w, (long)d.cd * d.K, SSM_INIT_UNIFORM, -kb, kb));
            SSM_TRY(I(L.conv_b, d.cd, SSM_INIT_UNIFORM, -kb, kb));
            SSM_TRY(I(L.dt_b, d.H, SSM_INIT_DT_BIAS, 1e-3f, 1e-1f));
            SSM_TRY(I(L.A_log, d.H, SSM_INIT_LOG_UNIFORM, 1.f, 16.f));
            SSM_TRY(I(L.Dsk, d.H, SSM_INIT_CONST, 1.f, 0.f));
            SSM_TRY(I(L.gnorm, d.D, SSM_INIT_CONST, 1.f, 0.f));
            SSM_TRY(I(L.out_proj, (long)d.d * d.D, SSM_INIT_NORMAL, 0.02f, 0.f));
        }
    }
    SSM_TRY(I(m->norm_f, d.d, SSM_INIT_CONST, 1.f, 0.f));
    return refresh_A(m);
}

// Workspace plan for T = B*L tokens (bytes, 256-aligned carve-outs).
struct Ws {
    float *hid, *nrm, *a, *b, *c, *d, *e, *last, *logits;
    // one-token steps (stepproj.hip): x * g of the next RMSNorm and the gated norm's output,
    // both in fragment order, and the two norms' partial sums of squares; null for longer
    // sequences (xg and ssq_in also hold the own LM head's operand, below)
    float *xg, *yf, *ssq_in, *ssq_y;
    // the Mamba-1 step's x_proj partials (stepproj.hip, xpart); null for longer sequences or
    // without Mamba-1 layers
    float* xpart;
    // the own LM head's argmax partials (head.hip), for its rows: all T positions when
    // T <= kStepProjMaxRows (one-token steps, short forwards), else a prefill's B last
    // positions when B <= kStepProjMaxRows; null otherwise
    float* hpart;
    // split-K partials of the own prefill GEMM (gemm.hip) for the largest split product of
    // the mixers at T tokens (gpart_n floats); null when none splits
    float* gpart;
    size_t gpart_n;
    void* scan;
    size_t scan_bytes;
};

size_t al(size_t b) { return (b + 255) & ~(size_t)255; }

size_t plan_ws(ssm_model* m, int B, int L, bool full_logits, Ws* out) {
    const Dims& d = m->dm;
    const size_t T = (size_t)B * L;
    size_t na = 0, nb = 0, nc = 0, ndd = 0, ne = 0, scan = 0;
    bool has1 = false, has2 = false;
    for (int t : m->types) (t == SSM_LAYER_MAMBA1 ? has1 : has2) = true;
    if (has1) {
        na = std::max(na, T * 2 * d.D);             // xz
        nb = std::max(nb, T * d.D);                 // xc
        nc = std::max(nc, T * (d.R + 2 * d.N));     // dbl
        ndd = std::max(ndd, T * d.D);               // dt
        ne = std::max(ne, T * d.D);                 // y
        scan = std::max(scan, ssm_selective_scan_workspace(B, L, d.D, d.N));
    }
    if (has2) {
        na = std::max(na, T * d.nin);               // zx
        nb = std::max(nb, T * d.cd);                // xbc
        nc = std::max(nc, T * d.D);                 // y
        ndd = std::max(ndd, T * d.D);               // yn
        scan = std::max(scan, ssm_ssd_workspace(B, L, d.H, d.P, d.G, d.N));
    }
    const size_t nlog = full_logits ? T * d.V : (size_t)B * d.V;
    size_t off = 0;
    size_t o_hid = off; off += al(4 * T * d.d);
    size_t o_nrm = off; off += al(4 * T * d.d);
    size_t o_a = off; off += al(4 * na);
    size_t o_b = off; off += al(4 * nb);
    size_t o_c = off; off += al(4 * nc);
    size_t o_d = off; off += al(4 * ndd);
    size_t o_e = off; off += al(4 * ne);
    size_t o_last = off; off += al(4 * (size_t)B * d.d);
    size_t o_log = off; off += al(4 * nlog);
    size_t o_scan = off; off += al(scan);
    const size_t nstep = L == 1 ? (size_t)B : 0;
    const size_t nstep16 = (nstep + 15) / 16 * 16;   // fragment order pads to 16-row tiles
    const size_t MR = ssm::kStepProjMaxRows;
    const size_t nhead = T <= MR ? T : (size_t)B <= MR ? (size_t)B : 0;
    const size_t nx = std::max(nstep, nhead), nx16 = (nx + 15) / 16 * 16;
    size_t o_xg = off; off += al(4 * nx16 * d.d);
    size_t o_yf = off; off += al(4 * nstep16 * d.D);
    size_t o_sqi = off; off += al(4 * nx * ssm::kStepProjMaxSsq);
    size_t o_sqy = off; off += al(4 * nstep * ssm::kStepProjMaxSsq);
    const size_t nxp = has1 ? (size_t)(d.D / 16) * nstep16 * (d.R + 2 * d.N) : 0;
    size_t o_xp = off; off += al(4 * nxp);
    const size_t nhp = nhead * (size_t)ssm::head_parts(d.V) * 2;
    size_t o_hp = off; off += al(4 * nhp);
    size_t ngp = 0;
    if (T >= (size_t)kOwnGemmRows && T <= (size_t)INT32_MAX) {
        const int t = (int)T;
        if (has1)
            for (auto nk : {std::pair<int, int>{2 * d.D, d.d}, {d.d, d.D}, {d.R + 2 * d.N, d.D},
                            {d.D, d.R}})
                ngp = std::max(ngp, ssm::gemm_split_floats(t, nk.first, nk.second));
        if (has2)
            for (auto nk : {std::pair<int, int>{d.nin, d.d}, {d.d, d.D}})
                ngp = std::max(ngp, ssm::gemm_split_floats(t, nk.first, nk.second));
    }
    size_t o_gp = off; off += al(4 * ngp);
    if (out) {
        char* base = m->ws;
        out->hid = (float*)(base + o_hid); out->nrm = (float*)(base + o_nrm);
        out->a = (float*)(base + o_a); out->b = (float*)(base + o_b);
        out->c = (float*)(base + o_c); out->d = (float*)(base + o_d);
        out->e = (float*)(base + o_e); out->last = (float*)(base + o_last);
        out->logits = (float*)(base + o_log);
        out->scan = base + o_scan; out->scan_bytes = scan;
        out->xg = nx ? (float*)(base + o_xg) : nullptr;
        out->yf = nstep ? (float*)(base + o_yf) : nullptr;
        out->ssq_in = nx ? (float*)(base + o_sqi) : nullptr;
        out->ssq_y = nstep ? (float*)(base + o_sqy) : nullptr;
        out->xpart = nxp ? (float*)(base + o_xp) : nullptr;
        out->hpart = nhp ? (float*)(base + o_hp) : nullptr;
        out->gpart = ngp ? (float*)(base + o_gp) : nullptr;
        out->gpart_n = ngp;
    }
    return off;
}

ssm_status ensure_ws(ssm_model* m, int B, int L, bool full_logits, Ws* w) {
    const size_t need = plan_ws(m, B, L, full_logits, nullptr);
    if (need > m->ws_bytes) {
        SSM_HIP_TRY(hipStreamSynchronize(m->ctx->stream));
        if (m->ws) SSM_HIP_TRY(hipFree(m->ws));
        m->ws = nullptr;
        m->ws_bytes = 0;
        SSM_HIP_TRY(ssm::dev_malloc((void**)&m->ws, need));
        m->ws_bytes = need;
    }
    plan_ws(m, B, L, full_logits, w);
    return SSM_OK;
}

ssm_status ensure_ids(ssm_model* m, size_t n) {
    if (n > m->ids_cap) {
        SSM_HIP_TRY(hipStreamSynchronize(m->ctx->stream));
        if (m->d_ids) SSM_HIP_TRY(hipFree(m->d_ids));
        m->d_ids = nullptr;
        SSM_HIP_TRY(ssm::dev_malloc((void**)&m->d_ids, n * sizeof(uint32_t)));
        m->ids_cap = n;
    }
    return SSM_OK;
}

bool al16(const void* p) { return ((uintptr_t)p & 15) == 0; }

ssm_status proj_rows(ssm_model* m, int mode, const float* x, long ldx, const float* z, long ldz,
                     const float* g, const float* W, float* y, long ldy, int M, int N, int K,
                     float beta, float* tmp, const float* g2 = nullptr, float* nout = nullptr,
                     bool* normed = nullptr, bool rows = false);

// One mixer over (B, L) tokens: reads x (T, d) [normalised], adds its output into out (T, d)
// with beta (0: overwrite, 1: residual add). ssm/conv state may be null (zero initial state).
// Its products: up to kFewRows tokens on the row kernel (proj_rows), else gemm() (the own
// kernel from kOwnGemmRows rows, with the split-K workspace).
ssm_status mixer(ssm_model* m, const LayerW& Ly, const float* x, float* out, float beta, int B,
                 int L, float* ssm_st, float* conv_st, const Ws& w) {
    const Dims& d = m->dm;
    ssm_ctx* c = m->ctx;
    hipStream_t st = c->stream;
    const int T = B * L;
    const float* W = m->w;
    const float* A = m->Ab + Ly.A;
    const bool few = few_rows(T);
    auto proj = [&](int N, int K, const float* X, long ldx, const float* Wt, float* Y, long ldy,
                    float b) -> ssm_status {
        if (few)
            return proj_rows(m, 0, X, ldx, nullptr, 0, nullptr, Wt, Y, ldy, T, N, K, b, nullptr,
                             nullptr, nullptr, nullptr, true);
        return gemm(c, T, N, K, X, ldx, Wt, Y, ldy, b, w.gpart, w.gpart_n);
    };
    if (Ly.type == SSM_LAYER_MAMBA1) {
        float *xz = w.a, *xc = w.b, *dbl = w.c, *dtv = w.d, *y = w.e;
        const int RN = d.R + 2 * d.N;
        // x_proj and dt_proj in one kernel when its workgroups (32 tokens each) cover the CUs;
        // with fewer tokens, two products (split over K by gemm()). With the fused kernel, the
        // scan's element-wise input work moves into its producers: in_proj stores silu(z) for
        // the z half and x_proj/dt_proj stores dt' = softplus(dt + bias) (the same functions,
        // so the same values).
        const bool fused_xd = own_kernels(T) && (T + 31) / 32 >= 256 &&
                              ssm::xproj_dt_ok(T, d.D, d.R, d.N, d.D, RN, d.D) &&
                              al16(W + Ly.x_proj) && al16(W + Ly.dt_w);
        const bool pre = fused_xd && ssm::gemm_ok(T, 2 * d.D, d.d, d.d, d.d, 2 * d.D) &&
                         al16(x) && al16(W + Ly.in_proj) && d.D % 16 == 0;
        { Stage g(c, "m1.in_proj");
          if (pre) SSM_TRY(ssm::launch_gemm(x, d.d, W + Ly.in_proj, d.d, nullptr, xz, 2 * d.D, T,
                                            2 * d.D, d.d, 0.f, st, nullptr, 0, 0.f, 0.f, d.D,
                                            w.gpart, w.gpart_n));
          else SSM_TRY(proj(2 * d.D, d.d, x, d.d, W + Ly.in_proj, xz, 2 * d.D, 0.f)); }
        { Stage g(c, "m1.conv");
          SSM_TRY(ssm_causal_conv1d(xz, 2 * d.D, W + Ly.conv_w, W + Ly.conv_b, xc, d.D, B, L, d.D,
                                    d.K, 1, conv_st, conv_st, st)); }
        if (fused_xd) {
            // x_proj and dt_proj in one pass (dt_low stays on chip)
            Stage g(c, "m1.x_dt_proj");
            SSM_TRY(ssm::launch_xproj_dt(xc, d.D, W + Ly.x_proj, W + Ly.dt_w, dbl, RN, dtv, d.D,
                                         T, d.D, d.R, d.N, st, pre ? W + Ly.dt_b : nullptr));
        } else {
            { Stage g(c, "m1.x_proj"); SSM_TRY(proj(RN, d.D, xc, d.D, W + Ly.x_proj, dbl, RN, 0.f)); }
            { Stage g(c, "m1.dt_proj"); SSM_TRY(proj(d.D, d.R, dbl, RN, W + Ly.dt_w, dtv, d.D, 0.f)); }
        }
        { Stage g(c, "m1.scan");
          SSM_TRY(ssm::selective_scan(xc, d.D, dtv, d.D, pre ? nullptr : W + Ly.dt_b, pre ? 0 : 1,
                                      A, dbl + d.R, RN, dbl + d.R + d.N, RN, W + Ly.Dsk, xz + d.D,
                                      2 * d.D, pre ? 1 : 0, y, d.D, B, L, d.D, d.N, ssm_st, ssm_st,
                                      w.scan, w.scan_bytes, st)); }
        { Stage g(c, "m1.out_proj"); SSM_TRY(proj(d.d, d.D, y, d.D, W + Ly.out_proj, out, d.d, beta)); }
    } else {
        float *zx = w.a, *xbc = w.b, *y = w.c, *yn = w.d;
        const int GN = d.G * d.N;
        { Stage g(c, "m2.in_proj"); SSM_TRY(proj(d.nin, d.d, x, d.d, W + Ly.in_proj, zx, d.nin, 0.f)); }
        { Stage g(c, "m2.conv");
          SSM_TRY(ssm_causal_conv1d(zx + d.D, d.nin, W + Ly.conv_w, W + Ly.conv_b, xbc, d.cd, B, L,
                                    d.cd, d.K, 1, conv_st, conv_st, st)); }
        const float* dtp = zx + d.D + d.cd;
        const bool fuse_gate =
            own_kernels(T) && ssm::gemm_ok(T, d.d, d.D, d.D, d.D, d.d) &&
            al16(W + Ly.out_proj) &&
            ssm::ssd_gated_ok(d.P, d.G, d.N, d.cd, d.nin, d.cd, d.cd, d.D, d.nin, xbc, xbc + d.D,
                              xbc + d.D + GN, y, zx, W + Ly.gnorm);
        if (fuse_gate) {
            // The gated RMSNorm split over its neighbours: the SSD stores u * g (u = y silu(z))
            // and per-head sums of u^2 (in yn's space), and out_proj scales each row by
            // 1 / rms(u) after the product.
            { Stage g(c, "m2.ssd_gate");
              SSM_TRY(ssm::ssd_f32(xbc, d.cd, dtp, d.nin, W + Ly.dt_b, 1, 0.f, INFINITY, A,
                                   xbc + d.D, d.cd, xbc + d.D + GN, d.cd, W + Ly.Dsk, y, d.D, B, L,
                                   d.H, d.G, d.N, ssm_st, ssm_st, w.scan, w.scan_bytes, st, zx,
                                   d.nin, W + Ly.gnorm, yn)); }
            { Stage g(c, "m2.out_proj");
              SSM_TRY(ssm::launch_gemm(y, d.D, W + Ly.out_proj, d.D, nullptr, out, d.d, T, d.d,
                                       d.D, beta, st, yn, d.H, 1.f / (float)d.D, d.eps,
                                       0x7fffffff, w.gpart, w.gpart_n)); }
        } else {
            { Stage g(c, "m2.ssd");
              SSM_TRY(ssm_ssd_chunk_scan(SSM_F32, xbc, d.cd, dtp, d.nin, W + Ly.dt_b, 1,
                                         0.f, INFINITY, A, xbc + d.D, d.cd, xbc + d.D + GN, d.cd,
                                         W + Ly.Dsk, y, d.D, B, L, d.H, d.P, d.G, d.N, ssm_st,
                                         ssm_st, w.scan, w.scan_bytes, st)); }
            if (few) {   // the gated norm in the row kernel's prologue
                Stage g(c, "m2.out_proj");
                SSM_TRY(proj_rows(m, 2, y, d.D, zx, d.nin, W + Ly.gnorm, W + Ly.out_proj, out,
                                  d.d, T, d.d, d.D, beta, yn, nullptr, nullptr, nullptr, true));
            } else {
                { Stage g(c, "m2.gated_norm");
                  SSM_TRY(ssm_gated_rmsnorm(y, d.D, zx, d.nin, W + Ly.gnorm, yn, d.D, T, d.D, d.G,
                                            d.eps, st)); }
                { Stage g(c, "m2.out_proj");
                  SSM_TRY(gemm(c, T, d.d, d.D, yn, d.D, W + Ly.out_proj, out, d.d, beta, w.gpart,
                               w.gpart_n)); }
            }
        }
    }
    return SSM_OK;
}

// The Mamba-2 mixer with bf16 operands and fp32 accumulation (one group, zero initial
// state): x, in_proj and out_proj weights, the SSD's x / B / C operands and out_proj's input
// are rounded to bf16 (round to nearest even); dt, the conv and the state pass stay fp32.
//   x -> bf16; in_proj: bf16 x bf16 -> fp32 zx (hipBLASLt); conv1d + SiLU on xBC -> bf16;
//   SSD on the bf16 operands (ssd.hip, v_mfma_f32_16x16x32_bf16) -> y fp32; gated RMSNorm
//   -> bf16; out_proj: bf16 x bf16 -> fp32 (hipBLASLt).
ssm_status mixer_bf16(ssm_model* m, int l, const float* x, float* out, int B, int L,
                      const Ws& w) {
    const Dims& d = m->dm;
    const LayerW& Ly = m->layers[l];
    ssm_ctx* c = m->ctx;
    hipStream_t st = c->stream;
    const int T = B * L;
    const float* W = m->w;
    const float* A = m->Ab + Ly.A;
    const int GN = d.G * d.N;
    SSM_REQUIRE(Ly.type == SSM_LAYER_MAMBA2, "bf16 mixer: layer %d is not a Mamba-2 layer", l);
    if (!m->wb) SSM_TRY(build_wb(m));
    __bf16* x16 = (__bf16*)w.hid;        // (T, d)
    float* zx = w.a;                     // (T, nin) fp32
    __bf16* xbc16 = (__bf16*)w.b;        // (T, cd)
    float* y = w.c;                      // (T, D) fp32
    __bf16* yn16 = (__bf16*)w.d;         // (T, D)
    { Stage g(c, "m2b.cast_x"); SSM_TRY(ssm::launch_cast_bf16(x, d.d, x16, d.d, T, d.d, st)); }
    { Stage g(c, "m2b.in_proj");
      SSM_TRY(gemm_bf16(c, T, d.nin, d.d, x16, d.d, m->wb + m->wb_in[l], zx, d.nin, 0.f)); }
    { Stage g(c, "m2b.conv");
      SSM_TRY(ssm::launch_conv1d_bf16(zx + d.D, d.nin, W + Ly.conv_w, W + Ly.conv_b, xbc16, d.cd,
                                      B, L, d.cd, d.K, 1, st)); }
    { Stage g(c, "m2b.ssd");
      SSM_TRY(ssm_ssd_chunk_scan(SSM_BF16, xbc16, d.cd, zx + d.D + d.cd, d.nin, W + Ly.dt_b, 1,
                                 0.f, INFINITY, A, xbc16 + d.D, d.cd, xbc16 + d.D + GN, d.cd,
                                 W + Ly.Dsk, y, d.D, B, L, d.H, d.P, d.G, d.N, nullptr, nullptr,
                                 w.scan, w.scan_bytes, st)); }
    { Stage g(c, "m2b.gated_norm");
      SSM_TRY(ssm::launch_gated_rmsnorm_bf16(y, d.D, zx, d.nin, W + Ly.gnorm, yn16, d.D, T, d.D,
                                             d.G, d.eps, st)); }
    { Stage g(c, "m2b.out_proj");
      SSM_TRY(gemm_bf16(c, T, d.d, d.D, yn16, d.D, m->wb + m->wb_out[l], out, d.d, 0.f)); }
    return SSM_OK;
}


// y (M, N) [ld ldy] = beta*y + s * p(x) W^T (mode 1: RMSNorm with weight g; mode 2: gated
// RMSNorm with z, one group): the few-row kernel (M <= 64) with the norm in its prologue
// where it is the faster choice, otherwise the norm as its own kernel into `tmp` and the
// library GEMM (gemm()). Measured at 64 rows (cfg4): the gated out_proj (N 1024, K 2048)
// 7.1 + 7.0 us split over K (the finish also writes the next layer's norm); the LM head
// (N 32000) 49 us with the norm fused, 70 us for norm + rocBLAS, about 42 us for norm +
// hipBLASLt; mode 1 below 16384 columns (in_proj) goes to the library GEMM.
//
// g2 / nout: when the few-row kernel's split finish can, it also writes nout = RMSNorm(y) * g2
// (the next layer's normalised input) and sets *normed.
ssm_status proj_rows(ssm_model* m, int mode, const float* x, long ldx, const float* z, long ldz,
                     const float* g, const float* W, float* y, long ldy, int M, int N, int K,
                     float beta, float* tmp, const float* g2, float* nout, bool* normed,
                     bool rows) {
    if (normed) *normed = false;
    ssm_ctx* c = m->ctx;
    const Dims& d = m->dm;
    // the LM head (RMS mode, wide N) takes RMSNorm + hipBLASLt when there is one (about 42
    // against 49 us at 64 x 32000 x 1024); the gated out_proj always takes the row kernel, and
    // so does every product when `rows` asks for it (the short prefill's)
    const bool wanted = rows || mode == 2 || (mode == 1 && N >= 16384 && !c->lt);
    const bool fits = wanted && ssm::rowgemm_ok(M, N, K) && al16(x) && al16(W) && ldx % 4 == 0 &&
                      al16(g) && (mode != 2 || (al16(z) && ldz % 4 == 0 && d.G == 1));
    if (fits) {
        const size_t need = ssm::rowgemm_workspace(M, N, K);
        if (need > m->rg_bytes) {
            SSM_HIP_TRY(hipStreamSynchronize(c->stream));
            if (m->rg) SSM_HIP_TRY(hipFree(m->rg));
            m->rg = nullptr;
            m->rg_bytes = 0;
            SSM_HIP_TRY(ssm::dev_malloc((void**)&m->rg, need));
            m->rg_bytes = need;
        }
        return ssm::launch_rowgemm(mode, x, ldx, z, ldz, g, W, y, ldy, M, N, K, beta, d.eps,
                                   m->rg, m->rg_bytes, c->stream, g2, nout, N, normed);
    }
    if (mode == 1) {
        SSM_TRY(ssm_rmsnorm(x, ldx, g, tmp, K, M, K, d.eps, c->stream));
        return gemm(c, M, N, K, tmp, K, W, y, ldy, beta);
    }
    if (mode == 2) {
        SSM_TRY(ssm_gated_rmsnorm(x, ldx, z, ldz, g, tmp, K, M, K, d.G, d.eps, c->stream));
        return gemm(c, M, N, K, tmp, K, W, y, ldy, beta);
    }
    return gemm(c, M, N, K, x, ldx, W, y, ldy, beta);
}

// One-token layer step for B sequences with the recurrent state:
// hid += mixer(RMSNorm(hid)). The norms ride in the projections' prologues (proj_rows).
//
// normed_in: w.nrm already holds RMSNorm(hid) * norm (the previous layer's out_proj wrote it);
// g_next: the next layer's norm weight, so that this layer's out_proj can write the next
// layer's normalised input into w.nrm (then *normed_out is set).
ssm_status mixer_step(ssm_model* m, const LayerW& Ly, float* hid, int B, float* ssm_st,
                      float* conv_st, const Ws& w, bool normed_in, const float* g_next,
                      bool* normed_out) {
    *normed_out = false;
    const Dims& d = m->dm;
    ssm_ctx* c = m->ctx;
    hipStream_t st = c->stream;
    const float* W = m->w;
    const float* A = m->Ab + Ly.A;
    if (Ly.type == SSM_LAYER_MAMBA1) {
        float *xz = w.a, *xc = w.b, *dbl = w.c, *dtv = w.d, *y = w.e;
        const int RN = d.R + 2 * d.N;
        { Stage g(c, "m1.step.in_proj");
          if (normed_in)
              SSM_TRY(gemm(c, B, 2 * d.D, d.d, w.nrm, d.d, W + Ly.in_proj, xz, 2 * d.D, 0.f));
          else
              SSM_TRY(proj_rows(m, 1, hid, d.d, nullptr, 0, W + Ly.norm, W + Ly.in_proj, xz,
                                2 * d.D, B, 2 * d.D, d.d, 0.f, w.nrm)); }
        { Stage g(c, "m1.step.conv");
          SSM_TRY(ssm_conv1d_update(xz, 2 * d.D, W + Ly.conv_w, W + Ly.conv_b, xc, d.D, conv_st, B,
                                    d.D, d.K, 1, st)); }
        { Stage g(c, "m1.step.x_proj");
          SSM_TRY(proj_rows(m, 0, xc, d.D, nullptr, 0, nullptr, W + Ly.x_proj, dbl, RN, B, RN,
                            d.D, 0.f, nullptr)); }
        { Stage g(c, "m1.step.dt_proj");
          SSM_TRY(proj_rows(m, 0, dbl, RN, nullptr, 0, nullptr, W + Ly.dt_w, dtv, d.D, B, d.D,
                            d.R, 0.f, nullptr)); }
        { Stage g(c, "m1.step.state_update");
          SSM_TRY(ssm_m1_state_update(xc, d.D, dtv, d.D, W + Ly.dt_b, 1, A, dbl + d.R, RN,
                                      dbl + d.R + d.N, RN, W + Ly.Dsk, xz + d.D, 2 * d.D, y, d.D,
                                      ssm_st, B, d.D, d.N, st)); }
        { Stage g(c, "m1.step.out_proj");
          SSM_TRY(proj_rows(m, 0, y, d.D, nullptr, 0, nullptr, W + Ly.out_proj, hid, d.d, B, d.d,
                            d.D, 1.f, nullptr)); }
    } else {
        float *zx = w.a, *xbc = w.b, *y = w.c, *yn = w.d;
        const int GN = d.G * d.N;
        { Stage g(c, "m2.step.in_proj");
          if (normed_in)
              SSM_TRY(gemm(c, B, d.nin, d.d, w.nrm, d.d, W + Ly.in_proj, zx, d.nin, 0.f));
          else
              SSM_TRY(proj_rows(m, 1, hid, d.d, nullptr, 0, W + Ly.norm, W + Ly.in_proj, zx,
                                d.nin, B, d.nin, d.d, 0.f, w.nrm)); }
        { Stage g(c, "m2.step.conv");
          SSM_TRY(ssm_conv1d_update(zx + d.D, d.nin, W + Ly.conv_w, W + Ly.conv_b, xbc, d.cd,
                                    conv_st, B, d.cd, d.K, 1, st)); }
        { Stage g(c, "m2.step.state_update");
          SSM_TRY(ssm_m2_state_update(xbc, d.cd, zx + d.D + d.cd, d.nin, W + Ly.dt_b, 1, 0.f,
                                      INFINITY, A, xbc + d.D, d.cd, xbc + d.D + GN, d.cd,
                                      W + Ly.Dsk, nullptr, 0, y, d.D, ssm_st, B, d.H, d.P, d.G,
                                      d.N, st)); }
        { Stage g(c, "m2.step.out_proj");
          SSM_TRY(proj_rows(m, 2, y, d.D, zx, d.nin, W + Ly.gnorm, W + Ly.out_proj, hid, d.d, B,
                            d.d, d.D, 1.f, yn, g_next, g_next ? w.nrm : nullptr, normed_out)); }
    }
    return SSM_OK;
}

// Whether a layer can take the fused one-token step: a Mamba-2 layer with one group whose
// projections fit the step kernel (stepproj.hip) and whose state update has a gated variant,
// or a Mamba-1 layer whose in_proj, x_proj and out_proj fit it (dt_proj is formed inside the
// state update).
bool fusable(const ssm_model* m, const LayerW& Ly) {
    const Dims& d = m->dm;
    if (Ly.type == SSM_LAYER_MAMBA1) {
        if (d.N > 64 || d.K > 8) return false;
        if (d.d % 16 != 0 || d.d / 16 > ssm::kStepProjMaxSsq) return false;
        // dt_proj rows as float4; the update's workgroups span 64 channels
        if (d.D % 64 != 0 || d.R % 4 != 0) return false;
        const int RN = d.R + 2 * d.N;
        return ssm::stepproj_ok(1, 2 * d.D, d.d) && ssm::stepproj_ok(1, RN, d.D) &&
               ssm::stepproj_ok(1, d.d, d.D);
    }
    if (Ly.type != SSM_LAYER_MAMBA2 || d.G != 1) return false;
    if (!(d.N == 64 || d.N == 128 || d.N == 256) || d.K > 8) return false;
    if (d.d % 16 != 0 || d.d / 16 > ssm::kStepProjMaxSsq) return false;
    if (ssm::m2_gated_nssq(d.H, d.P, d.N) > ssm::kStepProjMaxSsq) return false;
    if (d.D % 16 != 0 || d.cd % 4 != 0) return false;   // whole k-blocks; 16-byte B, C rows
    return ssm::stepproj_ok(1, d.nin, d.d) && ssm::stepproj_ok(1, d.d, d.D);
}

bool fused_step_ok(const ssm_model* m, const LayerW& Ly, int B, const Ws& w) {
    return B >= 1 && B <= ssm::kStepProjMaxRows && w.xg && w.yf && fusable(m, Ly);
}

// (Re)builds the fragment-order copies of the fusable layers' in_proj and out_proj.
ssm_status pack_weights(ssm_model* m) {
    const Dims& d = m->dm;
    hipStream_t st = m->ctx->stream;
    if (!m->wp) {
        long off = 0;
        m->wp_in.assign(d.nl, -1);
        m->wp_out.assign(d.nl, -1);
        m->wp_x.assign(d.nl, -1);
        m->wp_dt.assign(d.nl, -1);
        m->wp_xt.assign(d.nl, -1);
        const bool m1_step = ssm::m1_step_update_ok(d.D, d.N, d.R);
        for (int l = 0; l < d.nl; ++l) {
            if (!fusable(m, m->layers[l])) continue;
            if (m->layers[l].type == SSM_LAYER_MAMBA1) {
                m->wp_in[l] = off; off += (long)ssm::frag_floats(2 * d.D, d.d);
                m->wp_dt[l] = off; off += ((long)d.D * d.R + 63) / 64 * 64;
                if (m1_step) {   // x_proj rides in in_proj's epilogue: its transpose
                    m->wp_xt[l] = off;
                    off += ((long)d.D * (d.R + 2 * d.N) + 63) / 64 * 64;
                } else {         // x_proj is its own step projection
                    m->wp_x[l] = off;
                    off += (long)ssm::frag_floats(d.R + 2 * d.N, d.D);
                }
            } else {
                m->wp_in[l] = off; off += (long)ssm::frag_floats(d.nin, d.d);
            }
            m->wp_out[l] = off; off += (long)ssm::frag_floats(d.d, d.D);
        }
        if (ssm::head_ok(1, d.V, d.d)) {
            m->wp_emb = off;
            off += (long)ssm::frag_floats(d.V, d.d);
        }
        if (off == 0) return SSM_OK;
        SSM_HIP_TRY(ssm::dev_malloc((void**)&m->wp, (size_t)off * sizeof(float)));
    }
    for (int l = 0; l < d.nl; ++l) {
        if (m->wp_in[l] < 0) continue;
        const LayerW& Ly = m->layers[l];
        if (Ly.type == SSM_LAYER_MAMBA1) {
            const int RN = d.R + 2 * d.N;
            SSM_TRY(ssm::launch_pack_frag(m->w + Ly.in_proj, d.d, 2 * d.D, d.d,
                                          m->wp + m->wp_in[l], st));
            if (m->wp_x[l] >= 0)
                SSM_TRY(ssm::launch_pack_frag(m->w + Ly.x_proj, d.D, RN, d.D, m->wp + m->wp_x[l],
                                              st));
            // dt_proj is formed inside the state update: its rows in quads for the three-launch
            // step's update, else an aligned row-major copy
            if (m->wp_xt[l] >= 0) {
                SSM_TRY(ssm::launch_pack_q4(m->w + Ly.dt_w, d.D, d.R, m->wp + m->wp_dt[l], st));
                SSM_TRY(ssm::launch_pack_t(m->w + Ly.x_proj, d.D, RN, d.D, m->wp + m->wp_xt[l],
                                           st));
            } else {
                SSM_HIP_TRY(hipMemcpyAsync(m->wp + m->wp_dt[l], m->w + Ly.dt_w,
                                           sizeof(float) * (size_t)d.D * d.R,
                                           hipMemcpyDeviceToDevice, st));
            }
        } else {
            SSM_TRY(ssm::launch_pack_frag(m->w + Ly.in_proj, d.d, d.nin, d.d, m->wp + m->wp_in[l],
                                          st));
        }
        SSM_TRY(ssm::launch_pack_frag(m->w + Ly.out_proj, d.D, d.d, d.D, m->wp + m->wp_out[l],
                                      st));
    }
    if (m->wp_emb >= 0)
        SSM_TRY(ssm::launch_pack_frag(m->w + m->emb, d.d, d.V, d.d, m->wp + m->wp_emb, st));
    return SSM_OK;
}

// The fused one-token Mamba-1 layer step. Three launches when the state update can add x_proj's
// partials (ssm::m1_step_update_ok; the transposed x_proj is packed):
//   in_proj  (row scale 1/rms from w.ssq_in on w.xg = hid * norm) with the conv update of the
//            x columns in its epilogue: z into w.a (columns D .. 2D), SiLU(conv(x)) into w.b,
//            and x_proj summed over each 16-channel conv tile into w.xpart;
//   state update: x_proj's partials added per sequence, dt_proj (dt_r . W_dt[d], then bias and
//            softplus), the state, the D skip and the SiLU(z) gate; y in fragment order into
//            w.yf;
//   out_proj with the residual add into hid, and, given g_next, the next RMSNorm's operand
//            hid * g_next in w.xg and its partial sums in w.ssq_in.
// Otherwise four: in_proj also writes SiLU(conv(x)) in fragment order into w.yf, x_proj is a
// step projection of its own into w.c (dt_r, B, C), and the state update forms dt_proj from
// w.c.
// Same arithmetic as mixer_step up to the order of the norm's, x_proj's and dt_proj's sums
// and where the norm's scale is applied (the row scale multiplies the projected row).
ssm_status mixer_step_fused_m1(ssm_model* m, int l, float* hid, int B, float* ssm_st,
                               float* conv_st, const Ws& w, const float* g_next) {
    const Dims& d = m->dm;
    const LayerW& Ly = m->layers[l];
    ssm_ctx* c = m->ctx;
    hipStream_t st = c->stream;
    const float* W = m->w;
    const int RN = d.R + 2 * d.N;
    const bool three = m->wp_xt[l] >= 0 && w.xpart;
    float *xz = w.a, *xc = w.b, *dbl = w.c;
    { Stage g(c, "m1.step.in_proj");
      ssm::StepProj p;
      p.X = w.xg; p.W = m->wp + m->wp_in[l]; p.M = B; p.N = 2 * d.D; p.K = d.d;
      p.ssq = w.ssq_in; p.nssq = d.d / 16; p.inv_div = 1.f / (float)d.d; p.eps = d.eps;
      p.Y = xz; p.ldy = 2 * d.D;
      p.c0 = 0; p.C = d.D; p.Kc = d.K; p.cw = W + Ly.conv_w; p.cb = W + Ly.conv_b;
      p.cst = conv_st; p.Yc = xc; p.ldyc = d.D;
      if (three) {
          p.wxt = m->wp + m->wp_xt[l]; p.RN = RN; p.xpart = w.xpart;
      } else {
          p.Yf = w.yf;
      }
      SSM_TRY(ssm::launch_stepproj(ssm::EPI_CONV, p, st)); }
    if (three) {
        Stage g(c, "m1.step.state_update");
        SSM_TRY(ssm::launch_m1_step_update(xc, d.D, w.xpart, RN, (B + 15) / 16 * 16,
                                           m->wp + m->wp_dt[l], d.R, W + Ly.dt_b, m->Ab + Ly.A,
                                           W + Ly.Dsk, xz + d.D, 2 * d.D, w.yf, ssm_st, B, d.D,
                                           d.N, st));
    } else {
        { Stage g(c, "m1.step.x_proj");
          ssm::StepProj p;
          p.X = w.yf; p.W = m->wp + m->wp_x[l]; p.M = B; p.N = RN; p.K = d.D;
          p.Y = dbl; p.ldy = RN;
          SSM_TRY(ssm::launch_stepproj(ssm::EPI_STORE, p, st)); }
        { Stage g(c, "m1.step.state_update");
          SSM_TRY(ssm::launch_m1_update_frag(xc, d.D, dbl, RN, m->wp + m->wp_dt[l], d.R,
                                             W + Ly.dt_b, m->Ab + Ly.A, dbl + d.R, RN,
                                             dbl + d.R + d.N, RN, W + Ly.Dsk, xz + d.D,
                                             2 * d.D, w.yf, ssm_st, B, d.D, d.N, st)); }
    }
    { Stage g(c, "m1.step.out_proj");
      ssm::StepProj p;
      p.X = w.yf; p.W = m->wp + m->wp_out[l]; p.M = B; p.N = d.d; p.K = d.D;
      p.Y = hid; p.ldy = d.d;
      if (g_next) { p.g2 = g_next; p.xg = w.xg; p.ssq_out = w.ssq_in; }
      SSM_TRY(ssm::launch_stepproj(ssm::EPI_RESID, p, st)); }
    return SSM_OK;
}

// The fused one-token Mamba-2 layer step, three launches:
//   in_proj  (row scale 1/rms from w.ssq_in on w.xg = hid * norm) with the conv update of the
//            xBC columns in its epilogue: zx (z, dt) and xbc;
//   state update with the gated norm's element-wise part: w.yf = (C.h + D x) silu(z) gnorm
//            and the partial sums of ((C.h + D x) silu(z))^2 in w.ssq_y;
//   out_proj (row scale from w.ssq_y) with the residual add into hid, and, given g_next, the
//            next RMSNorm's operand hid * g_next in w.xg and its partial sums in w.ssq_in.
// Same arithmetic as mixer_step up to the order of the norms' sums and where each norm's
// scale is applied (the row scale multiplies the projected row).
ssm_status mixer_step_fused(ssm_model* m, int l, float* hid, int B, float* ssm_st,
                            float* conv_st, const Ws& w, const float* g_next) {
    const Dims& d = m->dm;
    const LayerW& Ly = m->layers[l];
    ssm_ctx* c = m->ctx;
    hipStream_t st = c->stream;
    const float* W = m->w;
    const float* A = m->Ab + Ly.A;
    if (Ly.type == SSM_LAYER_MAMBA1)
        return mixer_step_fused_m1(m, l, hid, B, ssm_st, conv_st, w, g_next);
    float *zx = w.a, *xbc = w.b;
    const int GN = d.G * d.N;
    { Stage g(c, "m2.step.in_proj");
      ssm::StepProj p;
      p.X = w.xg; p.W = m->wp + m->wp_in[l]; p.M = B; p.N = d.nin; p.K = d.d;
      p.ssq = w.ssq_in; p.nssq = d.d / 16; p.inv_div = 1.f / (float)d.d; p.eps = d.eps;
      p.Y = zx; p.ldy = d.nin;
      p.c0 = d.D; p.C = d.cd; p.Kc = d.K; p.cw = W + Ly.conv_w; p.cb = W + Ly.conv_b;
      p.cst = conv_st; p.Yc = xbc; p.ldyc = d.cd;
      SSM_TRY(ssm::launch_stepproj(ssm::EPI_CONV, p, st)); }
    { Stage g(c, "m2.step.state_update");
      SSM_TRY(ssm::launch_m2_update_gated(xbc, d.cd, zx + d.D + d.cd, d.nin, W + Ly.dt_b, A,
                                          xbc + d.D, d.cd, xbc + d.D + GN, d.cd, W + Ly.Dsk, zx,
                                          d.nin, W + Ly.gnorm, w.yf, w.ssq_y, ssm_st, B, d.H,
                                          d.P, d.G, d.N, st)); }
    { Stage g(c, "m2.step.out_proj");
      ssm::StepProj p;
      p.X = w.yf; p.W = m->wp + m->wp_out[l]; p.M = B; p.N = d.d; p.K = d.D;
      p.ssq = w.ssq_y; p.nssq = ssm::m2_gated_nssq(d.H, d.P, d.N);
      p.inv_div = 1.f / (float)d.D; p.eps = d.eps;
      p.Y = hid; p.ldy = d.d;
      if (g_next) { p.g2 = g_next; p.xg = w.xg; p.ssq_out = w.ssq_in; }
      SSM_TRY(ssm::launch_stepproj(ssm::EPI_RESID, p, st)); }
    return SSM_OK;
}

// embeddings -> layers; then the final norm into w.nrm unless `final_norm` is false (the
// one-token path, whose LM head applies it in its prologue: the result stays in w.hid). With
// `head_operand` (one-token steps into the own LM head), the final norm's operand hid * g_f and
// its partial sums go to w.xg / w.ssq_in instead: written by the last layer's out_proj when
// that layer takes the fused step, else by xg_ssq_kernel.
ssm_status trunk(ssm_model* m, const uint32_t* d_ids, int B, int L, ssm_state* s, const Ws& w,
                 bool final_norm = true, bool head_operand = false) {
    const Dims& d = m->dm;
    hipStream_t st = m->ctx->stream;
    const long T = (long)B * L;
    bool normed = false;   // w.nrm holds the next layer's normalised input (one-token path)
    bool pre = false;      // w.xg / w.ssq_in hold the next layer's x * g and partial sums
    if (L == 1 && s && d.nl > 0 && fused_step_ok(m, m->layers[0], B, w)) {
        // the first fused layer's norm operand comes with the embedding gather
        SSM_TRY(ssm::launch_embed_xg(d_ids, m->w + m->emb, w.hid, m->w + m->layers[0].norm,
                                     w.xg, w.ssq_in, B, d.d, d.V, m->d_flag, st));
        pre = true;
    } else {
        SSM_TRY(ssm::launch_embed(d_ids, m->w + m->emb, w.hid, T, d.d, d.V, m->d_flag, st));
    }
    for (int l = 0; l < d.nl; ++l) {
        const LayerW& Ly = m->layers[l];
        float* ss = s ? s->ssm[l] : nullptr;
        float* cs = s ? s->conv[l] : nullptr;
        if (L == 1 && s) {
            const LayerW* nx = l + 1 < d.nl ? &m->layers[l + 1] : nullptr;
            const bool next_fused = nx && fused_step_ok(m, *nx, B, w);
            if (fused_step_ok(m, Ly, B, w)) {
                if (!m->wp) SSM_TRY(pack_weights(m));   // eager: the first step never replays
                if (!pre)
                    SSM_TRY(ssm::launch_xg_ssq(w.hid, d.d, m->w + Ly.norm, w.xg, w.ssq_in, B, d.d,
                                               st));
                const bool last_op = !nx && head_operand;
                SSM_TRY(mixer_step_fused(m, l, w.hid, B, ss, cs, w,
                                         next_fused ? m->w + nx->norm
                                                    : last_op ? m->w + m->norm_f : nullptr));
                pre = next_fused || last_op;
                normed = false;
            } else {
                const float* g_next = nx && !next_fused ? m->w + nx->norm : nullptr;
                SSM_TRY(mixer_step(m, Ly, w.hid, B, ss, cs, w, normed, g_next, &normed));
                pre = false;
            }
        } else {
            SSM_TRY(ssm_rmsnorm(w.hid, d.d, m->w + Ly.norm, w.nrm, d.d, (int)T, d.d, d.eps, st));
            SSM_TRY(mixer(m, Ly, w.nrm, w.hid, 1.f, B, L, ss, cs, w));
        }
    }
    if (head_operand) {
        if (!pre || d.nl == 0)
            SSM_TRY(ssm::launch_xg_ssq(w.hid, d.d, m->w + m->norm_f, w.xg, w.ssq_in, B, d.d, st));
        return SSM_OK;
    }
    if (!final_norm) return SSM_OK;
    return ssm_rmsnorm(w.hid, d.d, m->w + m->norm_f, w.nrm, d.d, (int)T, d.d, d.eps, st);
}

// The own LM head (head.hip) over `rows` final hidden rows x (row stride ldx): the final
// norm's operand x * g_f in fragment order and its partial sums (xg_ssq_kernel), then the
// logits on the fragment-order tied embedding with the norm's scale applied per row, and the
// greedy picks into d_argmax when given. Replaces the final RMSNorm, the library product and
// the full-row argmax for up to kStepProjMaxRows rows.
bool own_head_ok(ssm_model* m, const Ws& w, long rows) {
    return w.xg && w.hpart && rows <= ssm::kStepProjMaxRows &&
           ssm::head_ok((int)rows, m->dm.V, m->dm.d);
}
ssm_status head_rows(ssm_model* m, const Ws& w, const float* x, long ldx, int rows, float* lg,
                     uint32_t* d_argmax) {
    const Dims& d = m->dm;
    hipStream_t st = m->ctx->stream;
    if (!m->wp) SSM_TRY(pack_weights(m));
    Stage g(m->ctx, "head");
    SSM_TRY(ssm::launch_xg_ssq(x, ldx, m->w + m->norm_f, w.xg, w.ssq_in, rows, d.d, st));
    return ssm::launch_head(w.xg, w.ssq_in, d.d / 16, 1.f / (float)d.d, d.eps,
                            m->wp + m->wp_emb, lg, d.V, rows, d.V, d.d, w.hpart, d_argmax, st);
}

ssm_status check_flag(ssm_model* m) {
    int bad = 0;
    SSM_HIP_TRY(hipMemcpyAsync(&bad, m->d_flag, sizeof(int), hipMemcpyDeviceToHost,
                               m->ctx->stream));
    SSM_HIP_TRY(hipStreamSynchronize(m->ctx->stream));
    if (bad) {
        SSM_HIP_TRY(hipMemsetAsync(m->d_flag, 0, sizeof(int), m->ctx->stream));
        return ssm::fail(SSM_ERR_INVALID_ARG, "token id out of range [0, %d)", m->dm.V);
    }
    return SSM_OK;
}

ssm_status validate_config(const ssm_config* cfg, Dims* out, std::vector<int>* types) {
    SSM_REQUIRE(cfg, "null config");
    Dims d{};
    d.V = cfg->vocab_size; d.d = cfg->d_model; d.nl = cfg->n_layers; d.N = cfg->d_state;
    d.K = cfg->d_conv; d.expand = cfg->expand; d.H = cfg->n_heads; d.G = cfg->n_groups;
    d.chunk = cfg->chunk_len; d.mimo = cfg->mimo_group; d.eos = cfg->eos_id;
    d.R = cfg->dt_rank > 0 ? cfg->dt_rank : (d.d + 15) / 16;
    d.eps = cfg->norm_eps > 0.f ? cfg->norm_eps : 1e-5f;
    SSM_REQUIRE(d.V > 0 && d.d > 0 && d.nl >= 0 && d.N > 0 && d.K >= 1 && d.K <= 8 &&
                    d.expand > 0 && d.H > 0 && d.G > 0,
                "config: non-positive dimension");
    // resolveModelConfig's own check (src/session/presets.ts:97-101)
    if (d.d % d.H != 0)
        return ssm::fail(SSM_ERR_INVALID_ARG, "dModel (%d) must be divisible by nHeads (%d).",
                         d.d, d.H);
    d.D = d.expand * d.d;
    d.P = d.D / d.H;
    d.cd = d.D + 2 * d.G * d.N;
    d.nin = 2 * d.D + 2 * d.G * d.N + d.H;
    types->assign(d.nl, SSM_LAYER_MAMBA1);
    for (int l = 0; l < d.nl; ++l) {
        const int t = cfg->layer_types ? cfg->layer_types[l] : SSM_LAYER_MAMBA1;
        if (t == SSM_LAYER_MAMBA1 || t == SSM_LAYER_MAMBA2) {
            (*types)[l] = t;
            continue;
        }
        return ssm::fail(SSM_ERR_UNSUPPORTED,
                         "layer %d: type %s is not implemented by the MI355X backend "
                         "(mamba1 and mamba2 are)", l,
                         t == SSM_LAYER_MAMBA3 ? "mamba3" : t == SSM_LAYER_ATTENTION ? "attention"
                                                                                   : "unknown");
    }
    for (int t : *types)
        if (t == SSM_LAYER_MAMBA2) {
            SSM_REQUIRE(d.H % d.G == 0, "nHeads (%d) must be divisible by nGroups (%d)", d.H, d.G);
            SSM_REQUIRE(d.N % 4 == 0, "mamba2 layers need dState divisible by 4");
        }
    *out = d;
    return SSM_OK;
}

}  // namespace

extern "C" ssm_status ssm_model_create(ssm_ctx* ctx, const ssm_config* cfg, uint64_t seed,
                                       ssm_model** out) {
    SSM_REQUIRE(out, "ssm_model_create: null out");
    *out = nullptr;
    CtxLock lk;
    SSM_TRY(ctx_enter(ctx, lk));
    ssm_model* m = new ssm_model();
    m->ctx = ctx;
    ssm_status s = validate_config(cfg, &m->dm, &m->types);
    if (s != SSM_OK) { delete m; return s; }
    build_layout(m);
    hipError_t e;
    if ((e = ssm::dev_malloc((void**)&m->w, m->nfloats * sizeof(float))) != hipSuccess ||
        (e = ssm::dev_malloc((void**)&m->Ab, (m->nA ? m->nA : 1) * sizeof(float))) != hipSuccess ||
        (e = ssm::dev_malloc((void**)&m->d_flag, sizeof(int))) != hipSuccess ||
        (e = hipMemsetAsync(m->d_flag, 0, sizeof(int), ctx->stream)) != hipSuccess) {
        hipFree(m->w); hipFree(m->Ab); hipFree(m->d_flag);
        delete m;
        return ssm::from_hip(e, "ssm_model_create");
    }
    s = random_init(m, seed);
    if (s == SSM_OK) {
        e = hipStreamSynchronize(ctx->stream);
        if (e != hipSuccess) s = ssm::from_hip(e, "ssm_model_create");
    }
    if (s != SSM_OK) {
        hipFree(m->w); hipFree(m->Ab); hipFree(m->d_flag);
        delete m;
        return s;
    }
    *out = m;
    return SSM_OK;
}

extern "C" ssm_status ssm_model_destroy(ssm_model* m) {
    if (!m) return SSM_OK;
    CtxLock lk(m->ctx->mu);
    if (m->destroyed) return SSM_OK;
    if (!m->ctx->destroyed) {
        hipSetDevice(m->ctx->device);
        hipStreamSynchronize(m->ctx->stream);
        hipFree(m->w); hipFree(m->Ab); hipFree(m->ws); hipFree(m->d_flag); hipFree(m->d_ids);
        hipFree(m->rg); hipFree(m->wp); hipFree(m->wb);
    }
    m->destroyed = true;
    return SSM_OK;
}

extern "C" ssm_status ssm_model_config(ssm_model* m, ssm_config* out) {
    CtxLock lk;
    SSM_TRY(model_enter(m, lk));
    SSM_REQUIRE(out, "null out");
    const Dims& d = m->dm;
    out->vocab_size = d.V; out->d_model = d.d; out->n_layers = d.nl; out->d_state = d.N;
    out->d_conv = d.K; out->expand = d.expand; out->n_heads = d.H; out->n_groups = d.G;
    out->chunk_len = d.chunk; out->mimo_group = d.mimo; out->eos_id = d.eos; out->dt_rank = d.R;
    out->norm_eps = d.eps;
    return SSM_OK;
}

namespace {
// The model's expectations of an SSMW image (ssmw.hpp).
ssmw::Expect ssmw_expect(const ssm_model* m, std::vector<unsigned char>& types) {
    const Dims& d = m->dm;
    types.assign(m->types.begin(), m->types.end());
    ssmw::Expect e{{d.V, d.d, d.nl, d.N, d.K, d.expand, d.H, d.G, d.R}, types.data(),
                   (uint64_t)m->nfloats};
    return e;
}
}  // namespace

extern "C" ssm_status ssm_model_export_weights(ssm_model* m, int f16, void* buf, size_t cap,
                                               size_t* bytes) {
    CtxLock lk;
    SSM_TRY(model_enter(m, lk));
    const size_t hb = ssmw::header_bytes(m->dm.nl);
    const size_t total = hb + m->nfloats * (f16 ? 2 : 4);
    if (bytes) *bytes = total;
    if (!buf) return SSM_OK;
    SSM_REQUIRE(cap >= total, "ssm_model_export_weights: buffer of %zu bytes needed", total);
    unsigned char* p = (unsigned char*)buf;
    std::vector<unsigned char> types;
    const ssmw::Expect e = ssmw_expect(m, types);
    const Dims& d = m->dm;
    ssmw::write_header(e.dims, d.eps, d.chunk, d.eos, d.mimo, e.layer_types, e.nfloats, f16, p);
    if (!f16) {
        SSM_HIP_TRY(hipMemcpyAsync(p + hb, m->w, m->nfloats * 4, hipMemcpyDeviceToHost,
                                   m->ctx->stream));
        SSM_HIP_TRY(hipStreamSynchronize(m->ctx->stream));
    } else {
        std::vector<float> tmp(m->nfloats);
        SSM_HIP_TRY(hipMemcpyAsync(tmp.data(), m->w, m->nfloats * 4, hipMemcpyDeviceToHost,
                                   m->ctx->stream));
        SSM_HIP_TRY(hipStreamSynchronize(m->ctx->stream));
        for (size_t i = 0; i < m->nfloats; ++i) {
            const uint16_t h = ssmw::f2h(tmp[i]);
            std::memcpy(p + hb + 2 * i, &h, 2);
        }
    }
    return SSM_OK;
}

extern "C" ssm_status ssm_model_load_weights(ssm_model* m, const void* buf, size_t bytes) {
    CtxLock lk;
    SSM_TRY(model_enter(m, lk));
    const unsigned char* p = (const unsigned char*)buf;
    std::vector<unsigned char> types;
    ssmw::Header h;
    if (const char* why = ssmw::validate(buf, bytes, ssmw_expect(m, types), &h))
        return ssm::fail(SSM_ERR_CHECKPOINT_INVALID, "%s", why);
    if (h.eps > 0.f) m->dm.eps = h.eps;
    if (h.dtype == 0) {
        SSM_HIP_TRY(hipMemcpyAsync(m->w, p + h.header_bytes, m->nfloats * 4,
                                   hipMemcpyHostToDevice, m->ctx->stream));
        SSM_HIP_TRY(hipStreamSynchronize(m->ctx->stream));
    } else {
        std::vector<float> tmp(m->nfloats);
        ssmw::decode_payload(p + h.header_bytes, h, tmp.data());
        SSM_HIP_TRY(hipMemcpyAsync(m->w, tmp.data(), m->nfloats * 4, hipMemcpyHostToDevice,
                                   m->ctx->stream));
        SSM_HIP_TRY(hipStreamSynchronize(m->ctx->stream));
    }
    SSM_TRY(refresh_A(m));
    SSM_HIP_TRY(hipStreamSynchronize(m->ctx->stream));
    return SSM_OK;
}

extern "C" ssm_status ssm_forward_device(ssm_model* m, const uint32_t* d_ids, int B, int L,
                                         float* d_logits) {
    CtxLock lk;
    SSM_TRY(model_enter(m, lk));
    SSM_REQUIRE(d_ids && d_logits && B >= 0 && L >= 0, "ssm_forward_device: bad args");
    if (B == 0 || L == 0) return SSM_OK;
    Ws w;
    SSM_TRY(ensure_ws(m, B, L, false, &w));
    const long T = (long)B * L;
    const bool own = own_head_ok(m, w, T);
    SSM_TRY(trunk(m, d_ids, B, L, nullptr, w, !own));
    if (own) return head_rows(m, w, w.hid, m->dm.d, (int)T, d_logits, nullptr);
    return gemm(m->ctx, B * L, m->dm.V, m->dm.d, w.nrm, m->dm.d, m->w + m->emb, d_logits,
                m->dm.V, 0.f);
}

extern "C" ssm_status ssm_forward(ssm_model* m, const uint32_t* ids, int B, int L,
                                  float* logits) {
    CtxLock lk;
    SSM_TRY(model_enter(m, lk));
    SSM_REQUIRE(ids && logits && B >= 0 && L >= 0, "ssm_forward: bad args");
    if (B == 0 || L == 0) return SSM_OK;
    const size_t T = (size_t)B * L;
    SSM_TRY(ensure_ids(m, T));
    Ws w;
    SSM_TRY(ensure_ws(m, B, L, true, &w));
    SSM_HIP_TRY(hipMemcpyAsync(m->d_ids, ids, T * 4, hipMemcpyHostToDevice, m->ctx->stream));
    const bool own = own_head_ok(m, w, (long)T);
    SSM_TRY(trunk(m, m->d_ids, B, L, nullptr, w, !own));
    if (own) SSM_TRY(head_rows(m, w, w.hid, m->dm.d, (int)T, w.logits, nullptr));
    else SSM_TRY(gemm(m->ctx, (int)T, m->dm.V, m->dm.d, w.nrm, m->dm.d, m->w + m->emb, w.logits,
                      m->dm.V, 0.f));
    SSM_HIP_TRY(hipMemcpyAsync(logits, w.logits, T * m->dm.V * 4, hipMemcpyDeviceToHost,
                               m->ctx->stream));
    return check_flag(m);
}

extern "C" ssm_status ssm_mixer_forward_device(ssm_model* m, int layer, const float* d_x,
                                               float* d_y, int B, int L) {
    CtxLock lk;
    SSM_TRY(model_enter(m, lk));
    SSM_REQUIRE(layer >= 0 && layer < m->dm.nl && d_x && d_y && B >= 0 && L >= 0,
                "ssm_mixer_forward_device: bad args");
    if (B == 0 || L == 0) return SSM_OK;
    Ws w;
    SSM_TRY(ensure_ws(m, B, L, false, &w));
    return mixer(m, m->layers[layer], d_x, d_y, 0.f, B, L, nullptr, nullptr, w);
}

extern "C" ssm_status ssm_mixer_forward_device_bf16(ssm_model* m, int layer, const float* d_x,
                                                    float* d_y, int B, int L) {
    CtxLock lk;
    SSM_TRY(model_enter(m, lk));
    SSM_REQUIRE(layer >= 0 && layer < m->dm.nl && d_x && d_y && B >= 0 && L >= 0,
                "ssm_mixer_forward_device_bf16: bad args");
    if (B == 0 || L == 0) return SSM_OK;
    Ws w;
    SSM_TRY(ensure_ws(m, B, L, false, &w));
    return mixer_bf16(m, layer, d_x, d_y, B, L, w);
}

// ------------------------------------------------------------------ state
extern "C" ssm_status ssm_state_create(ssm_model* m, int B, ssm_state** out) {
    SSM_REQUIRE(out, "ssm_state_create: null out");
    *out = nullptr;
    CtxLock lk;
    SSM_TRY(model_enter(m, lk));
    SSM_REQUIRE(B > 0, "ssm_state_create: batch must be positive");
    const Dims& d = m->dm;
    ssm_state* s = new ssm_state();
    s->m = m;
    s->B = B;
    size_t total = 0;
    for (int t : m->types) {
        const size_t a = t == SSM_LAYER_MAMBA1 ? (size_t)B * d.D * d.N : (size_t)B * d.H * d.P * d.N;
        const size_t c = (size_t)B * (t == SSM_LAYER_MAMBA1 ? d.D : d.cd) * (d.K - 1);
        s->ssm_n.push_back(a);
        s->conv_n.push_back(c);
        total += al(a * 4) / 4 + al(c * 4) / 4;
    }
    s->floats = 0;
    for (size_t i = 0; i < s->ssm_n.size(); ++i) s->floats += s->ssm_n[i] + s->conv_n[i];
    hipError_t e;
    if ((e = ssm::dev_malloc((void**)&s->buf, (total ? total : 1) * 4)) != hipSuccess ||
        (e = ssm::dev_malloc((void**)&s->d_tok, (size_t)B * 4)) != hipSuccess ||
        (e = ssm::dev_malloc((void**)&s->d_logits, (size_t)B * d.V * 4)) != hipSuccess) {
        hipFree(s->buf); hipFree(s->d_tok); hipFree(s->d_logits);
        delete s;
        return ssm::from_hip(e, "ssm_state_create");
    }
    size_t off = 0;
    for (size_t i = 0; i < s->ssm_n.size(); ++i) {
        s->ssm.push_back(s->buf + off); off += al(s->ssm_n[i] * 4) / 4;
        s->conv.push_back(s->buf + off); off += al(s->conv_n[i] * 4) / 4;
    }
    e = hipMemsetAsync(s->buf, 0, (total ? total : 1) * 4, m->ctx->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(m->ctx->stream);
    if (e != hipSuccess) {
        hipFree(s->buf); hipFree(s->d_tok); hipFree(s->d_logits);
        delete s;
        return ssm::from_hip(e, "ssm_state_create");
    }
    *out = s;
    return SSM_OK;
}

extern "C" ssm_status ssm_state_destroy(ssm_state* s) {
    if (!s) return SSM_OK;
    CtxLock lk(s->m->ctx->mu);
    if (s->destroyed) return SSM_OK;
    if (!s->m->destroyed && !s->m->ctx->destroyed) {
        hipSetDevice(s->m->ctx->device);
        hipStreamSynchronize(s->m->ctx->stream);
        for (auto& g : s->graphs)
            if (g.exec) hipGraphExecDestroy(g.exec);
        hipFree(s->buf); hipFree(s->d_tok); hipFree(s->d_logits); hipFree(s->d_gen);
        hipFree(s->d_ping); hipFree(s->d_u); hipFree(s->d_sws);
    }
    s->graphs.clear();
    s->destroyed = true;
    return SSM_OK;
}

extern "C" ssm_status ssm_state_reset(ssm_state* s) {
    CtxLock lk;
    SSM_TRY(state_enter(s, lk));
    for (size_t i = 0; i < s->ssm.size(); ++i) {
        SSM_HIP_TRY(hipMemsetAsync(s->ssm[i], 0, s->ssm_n[i] * 4, s->m->ctx->stream));
        SSM_HIP_TRY(hipMemsetAsync(s->conv[i], 0, s->conv_n[i] * 4, s->m->ctx->stream));
    }
    SSM_HIP_TRY(hipStreamSynchronize(s->m->ctx->stream));
    return SSM_OK;
}

extern "C" size_t ssm_state_floats(ssm_state* s) { return s ? s->floats : 0; }

extern "C" ssm_status ssm_state_read(ssm_state* s, float* out) {
    CtxLock lk;
    SSM_TRY(state_enter(s, lk));
    SSM_REQUIRE(out, "null out");
    size_t off = 0;
    for (size_t i = 0; i < s->ssm.size(); ++i) {
        SSM_HIP_TRY(hipMemcpyAsync(out + off, s->ssm[i], s->ssm_n[i] * 4, hipMemcpyDeviceToHost,
                                   s->m->ctx->stream));
        off += s->ssm_n[i];
        SSM_HIP_TRY(hipMemcpyAsync(out + off, s->conv[i], s->conv_n[i] * 4,
                                   hipMemcpyDeviceToHost, s->m->ctx->stream));
        off += s->conv_n[i];
    }
    SSM_HIP_TRY(hipStreamSynchronize(s->m->ctx->stream));
    return SSM_OK;
}

extern "C" ssm_status ssm_state_write(ssm_state* s, const float* in) {
    CtxLock lk;
    SSM_TRY(state_enter(s, lk));
    SSM_REQUIRE(in, "null in");
    size_t off = 0;
    for (size_t i = 0; i < s->ssm.size(); ++i) {
        SSM_HIP_TRY(hipMemcpyAsync(s->ssm[i], in + off, s->ssm_n[i] * 4, hipMemcpyHostToDevice,
                                   s->m->ctx->stream));
        off += s->ssm_n[i];
        SSM_HIP_TRY(hipMemcpyAsync(s->conv[i], in + off, s->conv_n[i] * 4,
                                   hipMemcpyHostToDevice, s->m->ctx->stream));
        off += s->conv_n[i];
    }
    SSM_HIP_TRY(hipStreamSynchronize(s->m->ctx->stream));
    return SSM_OK;
}

extern "C" ssm_status ssm_state_layer(ssm_state* s, int layer, float** ssm_p, float** conv_p) {
    CtxLock lk;
    SSM_TRY(state_enter(s, lk));
    SSM_REQUIRE(layer >= 0 && layer < (int)s->ssm.size(), "layer out of range");
    if (ssm_p) *ssm_p = s->ssm[layer];
    if (conv_p) *conv_p = s->conv[layer];
    return SSM_OK;
}

namespace {

// Prefill on device ids; leaves last-position logits in s->d_logits and argmax in d_argmax.
ssm_status prefill_device(ssm_model* m, ssm_state* s, const uint32_t* d_ids, int L,
                          uint32_t* d_argmax) {
    const Dims& d = m->dm;
    Ws w;
    SSM_TRY(ensure_ws(m, s->B, L, false, &w));
    // the own LM head on the B last positions (their final norm folded in), else the final
    // norm, the library product and the argmax
    const bool own = own_head_ok(m, w, s->B);
    SSM_TRY(trunk(m, d_ids, s->B, L, s, w, !own));
    if (own)
        return head_rows(m, w, w.hid + (long)(L - 1) * d.d, (long)L * d.d, s->B, s->d_logits,
                         d_argmax);
    SSM_TRY(ssm::launch_gather_rows(w.nrm, L, L - 1, w.last, s->B, d.d, m->ctx->stream));
    SSM_TRY(gemm(m->ctx, s->B, d.V, d.d, w.last, d.d, m->w + m->emb, s->d_logits, d.V, 0.f));
    if (d_argmax) SSM_TRY(ssm::launch_argmax(s->d_logits, d.V, s->B, d.V, d_argmax, m->ctx->stream));
    return SSM_OK;
}

ssm_status finish_host(ssm_model* m, ssm_state* s, float* logits, uint32_t* argmax,
                       const uint32_t* d_arg) {
    hipStream_t st = m->ctx->stream;
    if (logits)
        SSM_HIP_TRY(hipMemcpyAsync(logits, s->d_logits, (size_t)s->B * m->dm.V * 4,
                                   hipMemcpyDeviceToHost, st));
    if (argmax)
        SSM_HIP_TRY(hipMemcpyAsync(argmax, d_arg, (size_t)s->B * 4, hipMemcpyDeviceToHost, st));
    return check_flag(m);
}

ssm_status ensure_gen(ssm_state* s, size_t n) {
    if (n > s->gen_cap) {
        SSM_HIP_TRY(hipStreamSynchronize(s->m->ctx->stream));
        if (s->d_gen) SSM_HIP_TRY(hipFree(s->d_gen));
        s->d_gen = nullptr;
        SSM_HIP_TRY(ssm::dev_malloc((void**)&s->d_gen, n * 4));
        s->gen_cap = n;
    }
    return SSM_OK;
}

}  // namespace

extern "C" ssm_status ssm_prefill(ssm_model* m, ssm_state* s, const uint32_t* ids, int L,
                                  float* last_logits, uint32_t* argmax) {
    CtxLock lk;
    SSM_TRY(state_enter(s, lk));
    SSM_REQUIRE(s->m == m, "state belongs to another model");
    SSM_REQUIRE(ids && L > 0, "ssm_prefill: need at least one token");
    const size_t T = (size_t)s->B * L;
    SSM_TRY(ensure_ids(m, T));
    SSM_TRY(ensure_gen(s, (size_t)s->B));
    SSM_HIP_TRY(hipMemcpyAsync(m->d_ids, ids, T * 4, hipMemcpyHostToDevice, m->ctx->stream));
    SSM_TRY(prefill_device(m, s, m->d_ids, L, s->d_gen));
    return finish_host(m, s, last_logits, argmax, s->d_gen);
}

namespace {

ssm_status decode_body(ssm_model* m, ssm_state* s, const uint32_t* d_ids, float* lg,
                       uint32_t* d_argmax) {
    const Dims& d = m->dm;
    Ws w;
    SSM_TRY(ensure_ws(m, s->B, 1, false, &w));
    // the own LM head (head.hip) on the fragment-order embedding, with the final norm's scale
    // and the greedy pick folded in
    const bool own_head = w.xg && w.hpart && ssm::head_ok(s->B, d.V, d.d) && d.d % 16 == 0;
    if (own_head && !m->wp) SSM_TRY(pack_weights(m));   // eager: the first step never replays
    SSM_TRY(trunk(m, d_ids, s->B, 1, s, w, false, own_head));
    if (own_head) {
        Stage g(m->ctx, "head");
        return ssm::launch_head(w.xg, w.ssq_in, d.d / 16, 1.f / (float)d.d, d.eps,
                                m->wp + m->wp_emb, lg, d.V, s->B, d.V, d.d, w.hpart, d_argmax,
                                m->ctx->stream);
    }
    { Stage g(m->ctx, "head");
      SSM_TRY(proj_rows(m, 1, w.hid, d.d, nullptr, 0, m->w + m->norm_f, m->w + m->emb, lg, d.V,
                        s->B, d.V, d.d, 0.f, w.nrm)); }
    if (d_argmax) SSM_TRY(ssm::launch_argmax(lg, d.V, s->B, d.V, d_argmax, m->ctx->stream));
    return SSM_OK;
}

// Graph replay of repeated steps: off under the stage profiler (its events would be
// captured) and with SSM_DECODE_GRAPH=0.
bool graphs_on(const ssm_ctx* c) {
    if (c->prof) return false;
    const char* e = std::getenv("SSM_DECODE_GRAPH");
    return !(e && std::strcmp(e, "0") == 0);
}

constexpr size_t kMaxStepGraphs = 4;

// The first step with a set of pointers runs eagerly (it also grows any workspace the step
// needs, so none is allocated under capture); the second is captured and replayed, as are all
// later ones. The least recently used graph makes room for a new set.
ssm_status decode_graphed(ssm_model* m, ssm_state* s, const uint32_t* d_ids, float* lg,
                          uint32_t* d_argmax) {
    hipStream_t st = m->ctx->stream;
    ssm_state::StepGraph* e = nullptr;
    for (auto& g : s->graphs)
        if (g.ids == d_ids && g.logits == lg && g.argmax == d_argmax) e = &g;
    if (e && (e->ws != m->ws || e->rg != m->rg)) {   // a workspace moved: capture again
        if (e->exec) SSM_HIP_TRY(hipGraphExecDestroy(e->exec));
        e->exec = nullptr;
        e->ws = m->ws;
        e->rg = m->rg;
        return decode_body(m, s, d_ids, lg, d_argmax);
    }
    if (e && e->exec) {
        e->used = ++s->graph_clock;
        SSM_HIP_TRY(hipGraphLaunch(e->exec, st));
        return SSM_OK;
    }
    if (!e) {
        SSM_TRY(decode_body(m, s, d_ids, lg, d_argmax));
        if (s->graphs.size() >= kMaxStepGraphs) {
            auto old = std::min_element(s->graphs.begin(), s->graphs.end(),
                                        [](const auto& a, const auto& b) { return a.used < b.used; });
            if (old->exec) SSM_HIP_TRY(hipGraphExecDestroy(old->exec));
            s->graphs.erase(old);
        }
        s->graphs.push_back({d_ids, lg, d_argmax, m->ws, m->rg, nullptr, ++s->graph_clock});
        return SSM_OK;
    }
    hipGraph_t g = nullptr;
    SSM_HIP_TRY(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal));
    const ssm_status bs = decode_body(m, s, d_ids, lg, d_argmax);
    const hipError_t ce = hipStreamEndCapture(st, &g);
    if (bs != SSM_OK || ce != hipSuccess) {
        if (g) hipGraphDestroy(g);
        return bs != SSM_OK ? bs : ssm::from_hip(ce, "decode step capture");
    }
    hipGraphExec_t x = nullptr;
    const hipError_t ie = hipGraphInstantiate(&x, g, nullptr, nullptr, 0);
    hipGraphDestroy(g);
    SSM_HIP_TRY(ie);
    e->exec = x;
    e->ws = m->ws;
    e->rg = m->rg;
    e->used = ++s->graph_clock;
    SSM_HIP_TRY(hipGraphLaunch(x, st));
    return SSM_OK;
}

}  // namespace

extern "C" ssm_status ssm_decode_step_device(ssm_model* m, ssm_state* s, const uint32_t* d_ids,
                                             float* d_logits, uint32_t* d_argmax) {
    CtxLock lk;
    SSM_TRY(state_enter(s, lk));
    SSM_REQUIRE(s->m == m && d_ids, "ssm_decode_step_device: bad args");
    float* lg = d_logits ? d_logits : s->d_logits;
    if (!graphs_on(m->ctx)) return decode_body(m, s, d_ids, lg, d_argmax);
    return decode_graphed(m, s, d_ids, lg, d_argmax);
}

extern "C" ssm_status ssm_decode_step(ssm_model* m, ssm_state* s, const uint32_t* ids,
                                      float* logits, uint32_t* argmax) {
    CtxLock lk;
    SSM_TRY(state_enter(s, lk));
    SSM_REQUIRE(s->m == m && ids, "ssm_decode_step: bad args");
    SSM_TRY(ensure_gen(s, (size_t)s->B));
    SSM_HIP_TRY(hipMemcpyAsync(s->d_tok, ids, (size_t)s->B * 4, hipMemcpyHostToDevice,
                               m->ctx->stream));
    SSM_TRY(ssm_decode_step_device(m, s, s->d_tok, nullptr, s->d_gen));
    return finish_host(m, s, logits, argmax, s->d_gen);
}

namespace {

// Generation ring (n_new, B) on the device -> out_ids (B, n_new) on the host.
ssm_status gen_to_host(ssm_model* m, ssm_state* s, int n_new, uint32_t* out_ids) {
    const int B = s->B;
    std::vector<uint32_t> tmp((size_t)n_new * B);
    SSM_HIP_TRY(hipMemcpyAsync(tmp.data(), s->d_gen, tmp.size() * 4, hipMemcpyDeviceToHost,
                               m->ctx->stream));
    SSM_TRY(check_flag(m));
    for (int b = 0; b < B; ++b)
        for (int k = 0; k < n_new; ++k) out_ids[(size_t)b * n_new + k] = tmp[(size_t)k * B + b];
    return SSM_OK;
}

}  // namespace

extern "C" ssm_status ssm_generate_greedy(ssm_model* m, ssm_state* s, const uint32_t* prompt,
                                          int Lp, int n_new, uint32_t* out_ids) {
    CtxLock lk;
    SSM_TRY(state_enter(s, lk));
    SSM_REQUIRE(s->m == m && prompt && Lp > 0 && n_new >= 0 && (out_ids || n_new == 0),
                "ssm_generate_greedy: bad args");
    if (n_new == 0) return SSM_OK;
    const int B = s->B;
    const size_t T = (size_t)B * Lp;
    SSM_TRY(ensure_ids(m, T));
    SSM_TRY(ensure_gen(s, (size_t)n_new * B));
    hipStream_t st = m->ctx->stream;
    SSM_HIP_TRY(hipMemcpyAsync(m->d_ids, prompt, T * 4, hipMemcpyHostToDevice, st));
    SSM_TRY(prefill_device(m, s, m->d_ids, Lp, s->d_gen));
    // steps alternate between two id buffers (so they replay two captured graphs); each
    // step's argmax is then copied into the generation ring
    if (n_new > 1 && !s->d_ping) SSM_HIP_TRY(ssm::dev_malloc((void**)&s->d_ping, (size_t)2 * B * 4));
    if (n_new > 1)
        SSM_HIP_TRY(hipMemcpyAsync(s->d_ping, s->d_gen, (size_t)B * 4, hipMemcpyDeviceToDevice, st));
    for (int k = 1; k < n_new; ++k) {
        uint32_t* in = s->d_ping + (size_t)((k - 1) & 1) * B;
        uint32_t* outp = s->d_ping + (size_t)(k & 1) * B;
        SSM_TRY(ssm_decode_step_device(m, s, in, nullptr, outp));
        SSM_HIP_TRY(hipMemcpyAsync(s->d_gen + (size_t)k * B, outp, (size_t)B * 4,
                                   hipMemcpyDeviceToDevice, st));
    }
    return gen_to_host(m, s, n_new, out_ids);
}

extern "C" ssm_status ssm_generate_sample(ssm_model* m, ssm_state* s, const uint32_t* prompt,
                                          int Lp, int n_new, double temperature, int top_k,
                                          double top_p, const double* u_host,
                                          uint32_t* out_ids) {
    CtxLock lk;
    SSM_TRY(state_enter(s, lk));
    SSM_REQUIRE(s->m == m && prompt && Lp > 0 && n_new >= 0 &&
                    ((out_ids && u_host) || n_new == 0),
                "ssm_generate_sample: bad args");
    SSM_REQUIRE(top_k >= 1, "ssm_generate_sample: topK must be at least 1");
    if (!ssm::sample_ok(m->dm.V, top_k))
        return ssm::fail(SSM_ERR_UNSUPPORTED,
                         "ssm_generate_sample: vocabulary %d / topK %d beyond the device sampler",
                         m->dm.V, top_k);
    if (n_new == 0) return SSM_OK;
    const int B = s->B;
    const int V = m->dm.V;
    const size_t T = (size_t)B * Lp;
    const size_t nu = (size_t)n_new * B;
    SSM_TRY(ensure_ids(m, T));
    SSM_TRY(ensure_gen(s, nu));
    hipStream_t st = m->ctx->stream;
    if (nu > s->u_cap) {
        SSM_HIP_TRY(hipStreamSynchronize(st));
        if (s->d_u) SSM_HIP_TRY(hipFree(s->d_u));
        s->d_u = nullptr;
        SSM_HIP_TRY(ssm::dev_malloc((void**)&s->d_u, nu * sizeof(double)));
        s->u_cap = nu;
    }
    if (!s->d_sws) SSM_HIP_TRY(ssm::dev_malloc(&s->d_sws, ssm::sample_workspace(B, V)));
    SSM_HIP_TRY(hipMemcpyAsync(s->d_u, u_host, nu * sizeof(double), hipMemcpyHostToDevice, st));
    SSM_HIP_TRY(hipMemcpyAsync(m->d_ids, prompt, T * 4, hipMemcpyHostToDevice, st));
    SSM_TRY(prefill_device(m, s, m->d_ids, Lp, nullptr));
    SSM_TRY(ssm::launch_sample(s->d_logits, V, B, V, temperature, top_k, top_p, s->d_u,
                               s->d_gen, s->d_sws, st));
    // as in greedy generation, steps alternate between two id buffers so that they replay
    // two captured graphs; the sampler runs after each step, outside the graph (its draws
    // change every step)
    if (n_new > 1 && !s->d_ping) SSM_HIP_TRY(ssm::dev_malloc((void**)&s->d_ping, (size_t)2 * B * 4));
    if (n_new > 1)
        SSM_HIP_TRY(hipMemcpyAsync(s->d_ping, s->d_gen, (size_t)B * 4, hipMemcpyDeviceToDevice, st));
    for (int k = 1; k < n_new; ++k) {
        uint32_t* in = s->d_ping + (size_t)((k - 1) & 1) * B;
        uint32_t* outp = s->d_ping + (size_t)(k & 1) * B;
        SSM_TRY(ssm_decode_step_device(m, s, in, nullptr, nullptr));
        SSM_TRY(ssm::launch_sample(s->d_logits, V, B, V, temperature, top_k, top_p,
                                   s->d_u + (size_t)k * B, outp, s->d_sws, st));
        SSM_HIP_TRY(hipMemcpyAsync(s->d_gen + (size_t)k * B, outp, (size_t)B * 4,
                                   hipMemcpyDeviceToDevice, st));
    }
    return gen_to_host(m, s, n_new, out_ids);
}
