// C ABI of the int4 x int8 path (include/webyiq_q4q8.h).
//
// Every entry point validates its arguments on the host first and returns a
// status code with a thread-local message, like the engine's
// Result<_, String> (webyIQ crates/engine/src/graph.rs:186-222,368-380,
// manifest.rs:82-84).  Nothing is launched when validation fails, so all
// error paths are exercisable without a GPU.
#include <stdarg.h>
#include <stdio.h>

#include <atomic>
#include <mutex>
#include <string>

#include "../../include/webyiq_q4q8.h"
#include "launch.hpp"

namespace {

thread_local std::string g_err;

int fail(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_err = buf;
    return code;
}

int ok() {
    g_err.clear();
    return WQ_OK;
}

int hip_status(hipError_t e, const char* what) {
    if (e != hipSuccess) return fail(WQ_EHIP, "%s: %s", what, hipGetErrorString(e));
    return ok();
}

bool aligned(const void* p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

// Scratch of wq_lm_head_argmax_noalloc: the cross-workgroup argmax slots
// (keys and tickets, the layout of the caller-provided workspace of
// wq_lm_head_argmax), one copy per GPU for the life of the process.  Static
// device memory starts zeroed when the code object loads, and every call
// leaves it zeroed again.  The host never names the array in a launch: its
// device address comes from hipGetSymbolAddress, once per device.
static __device__ __align__(256) unsigned char scratch[wq::kArgmaxWorkspaceBytes];

constexpr int kMaxDevices = 64;
std::atomic<void*> g_scratch_ptr[kMaxDevices];
std::mutex g_scratch_mu;

// Device address of `scratch` on the current device (looked up on the first
// call per device, with that device current).
hipError_t scratch_ptr(void** out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
    void* p = g_scratch_ptr[dev].load(std::memory_order_acquire);
    if (!p) {
        std::lock_guard<std::mutex> lock(g_scratch_mu);
        p = g_scratch_ptr[dev].load(std::memory_order_relaxed);
        if (!p) {
            e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
            if (e != hipSuccess) return e;
            if (!p) return hipErrorInvalidSymbol;
            g_scratch_ptr[dev].store(p, std::memory_order_release);
        }
    }
    *out = p;
    return hipSuccess;
}

#define REQUIRE_PTR(p)                                                   \
    do {                                                                 \
        if (!(p)) return fail(WQ_EINVAL, "%s: %s is NULL", fn, #p);      \
    } while (0)
#define REQUIRE_ALIGN(p, a)                                                              \
    do {                                                                                 \
        if (!aligned((p), (a))) return fail(WQ_EALIGN, "%s: %s not %d-byte aligned", fn, \
                                            #p, (int)(a));                               \
    } while (0)

// Group / granularity rules shared by the quantiser and the products
// (graph.rs:378 requires K % 128; manifest.rs:82 fixed G = 32, G = 128 added).
int check_groups(const char* fn, int64_t K, int32_t G, int32_t GA) {
    if (K < 128 || K % 128 != 0)
        return fail(WQ_ESHAPE, "%s: K = %lld must be a positive multiple of 128", fn, (long long)K);
    if (G != 32 && G != 128)
        return fail(WQ_ESHAPE, "%s: unsupported quant group G = %d (32 or 128)", fn, G);
    if (GA != 32 && (int64_t)GA != K)
        return fail(WQ_ESHAPE, "%s: activation group GA = %d must be 32 or K = %lld", fn, GA,
                    (long long)K);
    return WQ_OK;
}

int check_linear(const char* fn, const uint32_t* wq, const uint32_t* ws, int64_t N, int64_t K,
                 int32_t G, const int8_t* xq, const float* dx, const int32_t* xs, int64_t M,
                 int32_t GA, int32_t mode, const float* y, bool need_y) {
    REQUIRE_PTR(wq);
    REQUIRE_PTR(ws);
    REQUIRE_PTR(xq);
    REQUIRE_PTR(dx);
    REQUIRE_PTR(xs);
    if (need_y) REQUIRE_PTR(y);
    if (mode < WQ_MODE_STORE || mode > WQ_MODE_SILU_MUL)
        return fail(WQ_EINVAL, "%s: unknown mode %d", fn, mode);
    if (N < 1 || N > (int64_t(1) << 30))
        return fail(WQ_ESHAPE, "%s: N = %lld out of range", fn, (long long)N);
    if (M < 1 || M > (int64_t(1) << 30))
        return fail(WQ_ESHAPE, "%s: M = %lld out of range", fn, (long long)M);
    int rc = check_groups(fn, K, G, GA);
    if (rc) return rc;
    REQUIRE_ALIGN(wq, 16);
    REQUIRE_ALIGN(xq, 16);
    REQUIRE_ALIGN(ws, 4);
    REQUIRE_ALIGN(dx, 4);
    REQUIRE_ALIGN(xs, 4);
    if (y) REQUIRE_ALIGN(y, 4);
    return WQ_OK;
}

// The decode GEMV keeps <= 8 tokens in registers and <= 8 passes of 2048
// codes per row (one workgroup of <= 16 waves).
int check_gemv_shape(const char* fn, int64_t M, int64_t K) {
    if (M > wq::kGemvMaxTokens)
        return fail(WQ_ESHAPE, "%s: M = %lld tokens exceeds the decode GEMV limit of %d", fn,
                    (long long)M, wq::kGemvMaxTokens);
    if (K > 8 * wq::kGemvPassK)
        return fail(WQ_ESHAPE, "%s: K = %lld exceeds the decode GEMV limit of %d", fn,
                    (long long)K, 8 * wq::kGemvPassK);
    return WQ_OK;
}

wq::LinearArgs make_args(const uint32_t* wq, const uint32_t* ws, int64_t N, int64_t K, int32_t G,
                         const int8_t* xq, const float* dx, const int32_t* xs, int64_t M,
                         int32_t GA, int32_t mode, float* y, int32_t* acc,
                         const wq_params* params = nullptr) {
    wq::LinearArgs a{};
    a.wq = wq;
    a.ws = ws;
    a.N = N;
    a.K = K;
    a.G = G;
    a.xq = xq;
    a.dx = dx;
    a.xs = xs;
    a.M = M;
    a.GA = GA;
    a.mode = mode;
    a.y = y;
    a.acc_dump = acc;
    a.params = reinterpret_cast<const uint32_t*>(params);
    return a;
}

int gemv_impl(const char* fn, void* stream, const uint32_t* wq, const uint32_t* ws, int64_t N,
              int64_t K, int32_t G, const int8_t* xq, const float* dx, const int32_t* xs,
              int64_t M, int32_t GA, int32_t mode, float* y, int32_t* acc) {
    int rc = check_linear(fn, wq, ws, N, K, G, xq, dx, xs, M, GA, mode, y, true);
    if (rc) return rc;
    rc = check_gemv_shape(fn, M, K);
    if (rc) return rc;
    auto a = make_args(wq, ws, N, K, G, xq, dx, xs, M, GA, mode, y, acc);
    return hip_status(wq::launch_gemv(a, static_cast<hipStream_t>(stream)), fn);
}

int gemm_impl(const char* fn, void* stream, const uint32_t* wq, const uint32_t* ws, int64_t N,
              int64_t K, int32_t G, const int8_t* xq, const float* dx, const int32_t* xs,
              int64_t M, int32_t GA, int32_t mode, float* y, int32_t* acc,
              const wq_params* params = nullptr, void* workspace = nullptr, size_t workspace_bytes = 0) {
    int rc = check_linear(fn, wq, ws, N, K, G, xq, dx, xs, M, GA, mode, y, true);
    if (rc) return rc;
    // the GEMM stages tiles with 32-bit byte offsets from each operand's base
    const int64_t rows = mode == WQ_MODE_SILU_MUL ? 2 * N : N;
    const int64_t lim = int64_t(0xFFFFFFFF);
    if (M * K > lim || rows * (K / 2) > lim)
        return fail(WQ_ESHAPE, "%s: M = %lld, rows = %lld, K = %lld address more than 4 GiB of one operand; "
                    "split the call along M or N", fn, (long long)M, (long long)rows, (long long)K);
    if (params) REQUIRE_ALIGN(params, 4);
    if (workspace) REQUIRE_ALIGN(workspace, 256);
    auto a = make_args(wq, ws, N, K, G, xq, dx, xs, M, GA, mode, y, acc, params);
    a.workspace = workspace;
    a.workspace_bytes = workspace ? workspace_bytes : 0;
    return hip_status(wq::launch_gemm(a, static_cast<hipStream_t>(stream)), fn);
}

}  // namespace

extern "C" {

const char* wq_last_error(void) { return g_err.c_str(); }

int wq_abi_version(void) { return WQ_ABI_VERSION; }

int wq_quant_act(void* stream, const float* x, const float* norm_w, float eps, int64_t M,
                 int64_t K, int32_t GA, int32_t G, int8_t* xq, float* dx, int32_t* xs) {
    const char* fn = "wq_quant_act";
    REQUIRE_PTR(x);
    REQUIRE_PTR(xq);
    REQUIRE_PTR(dx);
    REQUIRE_PTR(xs);
    if (M < 1 || M > (int64_t(1) << 30))
        return fail(WQ_ESHAPE, "%s: M = %lld out of range", fn, (long long)M);
    int rc = check_groups(fn, K, G, GA);
    if (rc) return rc;
    if (K > (int64_t(1) << 24)) return fail(WQ_ESHAPE, "%s: K = %lld too large", fn, (long long)K);
    REQUIRE_ALIGN(x, 16);
    if (norm_w) REQUIRE_ALIGN(norm_w, 16);
    REQUIRE_ALIGN(xq, 16);
    REQUIRE_ALIGN(dx, 4);
    REQUIRE_ALIGN(xs, 4);
    if (norm_w && !(eps >= 0.0f)) return fail(WQ_EINVAL, "%s: eps must be >= 0", fn);
    wq::QuantArgs a{x, norm_w, eps, M, K, GA, G, xq, dx, xs};
    return hip_status(wq::launch_quant_act(a, static_cast<hipStream_t>(stream)), fn);
}

int wq_gemv(void* stream, const uint32_t* wq, const uint32_t* ws, int64_t N, int64_t K, int32_t G,
            const int8_t* xq, const float* dx, const int32_t* xs, int64_t M, int32_t GA,
            int32_t mode, float* y) {
    return gemv_impl("wq_gemv", stream, wq, ws, N, K, G, xq, dx, xs, M, GA, mode, y, nullptr);
}

int wq_quant_gemv(void* stream, const float* x, const float* norm_w, float eps, const uint32_t* wq,
                  const uint32_t* ws, int64_t N, int64_t K, int32_t G, int64_t M, int32_t mode,
                  int8_t* xq, float* dx, int32_t* xs, float* y) {
    const char* fn = "wq_quant_gemv";
    REQUIRE_PTR(x);
    int rc = check_gemv_shape(fn, M, K);
    if (rc) return rc;
    rc = check_linear(fn, wq, ws, N, K, G, xq, dx, xs, M, (int32_t)K, mode, y, true);
    if (rc) return rc;
    REQUIRE_ALIGN(x, 16);
    if (norm_w) REQUIRE_ALIGN(norm_w, 16);
    if (norm_w && !(eps >= 0.0f)) return fail(WQ_EINVAL, "%s: eps must be >= 0", fn);
    auto a = make_args(wq, ws, N, K, G, xq, dx, xs, M, (int32_t)K, mode, y, nullptr);
    hipStream_t st = static_cast<hipStream_t>(stream);
    if (M <= 2) {  // one launch: every workgroup quantises while its weights stream in
        wq::QuantInArgs q{x, norm_w, eps, xq, dx, xs};
        return hip_status(wq::launch_gemv_quant_in(a, q, st), fn);
    }
    wq::QuantArgs qa{x, norm_w, eps, M, K, (int32_t)K, G, xq, dx, xs};
    rc = hip_status(wq::launch_quant_act(qa, st), fn);
    if (rc) return rc;
    return hip_status(wq::launch_gemv(a, st), fn);
}

int wq_gemm(void* stream, const uint32_t* wq, const uint32_t* ws, int64_t N, int64_t K, int32_t G,
            const int8_t* xq, const float* dx, const int32_t* xs, int64_t M, int32_t GA,
            int32_t mode, float* y, const wq_params* params, void* workspace, size_t workspace_bytes) {
    return gemm_impl("wq_gemm", stream, wq, ws, N, K, G, xq, dx, xs, M, GA, mode, y, nullptr, params, workspace,
                     workspace_bytes);
}

size_t wq_gemm_workspace_bytes(int64_t N, int64_t K, int32_t G, int64_t M, int32_t GA, int32_t mode) {
    if (N < 1 || M < 1 || K < 128 || K % 128 != 0 || (G != 32 && G != 128) || mode < 0 || mode > 2) return 0;
    wq::LinearArgs a{};
    a.N = N;
    a.K = K;
    a.G = G;
    a.M = M;
    a.GA = GA;
    a.mode = mode;
    return wq::gemm_workspace_bytes(a);
}

int wq_gemv_debug_acc(void* stream, const uint32_t* wq, const uint32_t* ws, int64_t N, int64_t K,
                      int32_t G, const int8_t* xq, const float* dx, const int32_t* xs, int64_t M,
                      int32_t GA, int32_t mode, float* y, int32_t* acc) {
    const char* fn = "wq_gemv_debug_acc";
    REQUIRE_PTR(acc);
    return gemv_impl(fn, stream, wq, ws, N, K, G, xq, dx, xs, M, GA, mode, y, acc);
}

int wq_gemm_debug_acc(void* stream, const uint32_t* wq, const uint32_t* ws, int64_t N, int64_t K,
                      int32_t G, const int8_t* xq, const float* dx, const int32_t* xs, int64_t M,
                      int32_t GA, int32_t mode, float* y, int32_t* acc) {
    const char* fn = "wq_gemm_debug_acc";
    REQUIRE_PTR(acc);
    return gemm_impl(fn, stream, wq, ws, N, K, G, xq, dx, xs, M, GA, mode, y, acc);
}

int wq_matmul(void* stream, int32_t path, const uint32_t* wq, const uint32_t* ws, int64_t N,
              int64_t K, int32_t G, const int8_t* xq, const float* dx, const int32_t* xs,
              int64_t M, int32_t GA, int32_t mode, float* y, const wq_params* params) {
    const char* fn = "wq_matmul";
    switch (path) {
        case WQ_PATH_PREFILL:
            return gemm_impl(fn, stream, wq, ws, N, K, G, xq, dx, xs, M, GA, mode, y, nullptr, params);
        case WQ_PATH_DECODE:
            if (M != 1) return fail(WQ_ESHAPE, "%s: decode path takes M = 1, got %lld", fn, (long long)M);
            return gemv_impl(fn, stream, wq, ws, N, K, G, xq, dx, xs, M, GA, mode, y, nullptr);
        case WQ_PATH_SPEC:
            return gemv_impl(fn, stream, wq, ws, N, K, G, xq, dx, xs, M, GA, mode, y, nullptr);
        default:
            return fail(WQ_EINVAL, "%s: unknown path %d", fn, path);
    }
}

int wq_argmax(void* stream, const float* logits, int64_t M, int64_t V, const uint32_t* ids,
              uint32_t* tok_out) {
    const char* fn = "wq_argmax";
    REQUIRE_PTR(logits);
    REQUIRE_PTR(tok_out);
    if (M < 1 || M > (int64_t(1) << 30))
        return fail(WQ_ESHAPE, "%s: M = %lld out of range", fn, (long long)M);
    if (V < 1 || V > (int64_t)0xFFFFFFFEll)
        return fail(WQ_ESHAPE, "%s: V = %lld out of range", fn, (long long)V);
    REQUIRE_ALIGN(logits, 4);
    REQUIRE_ALIGN(tok_out, 4);
    return hip_status(wq::launch_argmax(logits, M, V, ids, tok_out, static_cast<hipStream_t>(stream)), fn);
}

int wq_embed(void* stream, const uint32_t* eq, const uint32_t* es, int64_t V, int64_t K, int32_t G,
             const uint32_t* tok, int64_t M, float* x) {
    const char* fn = "wq_embed";
    REQUIRE_PTR(eq);
    REQUIRE_PTR(es);
    REQUIRE_PTR(tok);
    REQUIRE_PTR(x);
    if (V < 1 || V > (int64_t)0xFFFFFFFFll)
        return fail(WQ_ESHAPE, "%s: V = %lld out of range", fn, (long long)V);
    if (M < 1 || M > (int64_t(1) << 30))
        return fail(WQ_ESHAPE, "%s: M = %lld out of range", fn, (long long)M);
    int rc = check_groups(fn, K, G, (int32_t)K);
    if (rc) return rc;
    REQUIRE_ALIGN(eq, 16);
    REQUIRE_ALIGN(es, 4);
    REQUIRE_ALIGN(tok, 4);
    REQUIRE_ALIGN(x, 16);
    wq::EmbedArgs a{eq, es, V, K, G, tok, M, x};
    return hip_status(wq::launch_embed(a, static_cast<hipStream_t>(stream)), fn);
}

int wq_gather_rows(void* stream, const uint32_t* sq, const uint32_t* ss, int64_t V, int64_t K,
                   int32_t G, const uint32_t* ids, int64_t R, uint32_t* dq, uint32_t* ds) {
    const char* fn = "wq_gather_rows";
    REQUIRE_PTR(sq);
    REQUIRE_PTR(ss);
    REQUIRE_PTR(ids);
    REQUIRE_PTR(dq);
    REQUIRE_PTR(ds);
    if (V < 1 || V > (int64_t)0xFFFFFFFFll)
        return fail(WQ_ESHAPE, "%s: V = %lld out of range", fn, (long long)V);
    if (R < 1 || R > (int64_t(1) << 30))
        return fail(WQ_ESHAPE, "%s: R = %lld out of range", fn, (long long)R);
    int rc = check_groups(fn, K, G, (int32_t)K);
    if (rc) return rc;
    REQUIRE_ALIGN(sq, 16);
    REQUIRE_ALIGN(dq, 16);
    REQUIRE_ALIGN(ss, 4);
    REQUIRE_ALIGN(ds, 4);
    REQUIRE_ALIGN(ids, 4);
    wq::GatherArgs a{sq, ss, V, K, G, ids, R, dq, ds};
    return hip_status(wq::launch_gather_rows(a, static_cast<hipStream_t>(stream)), fn);
}

int wq_mtp_in(void* stream, const float* emb, const float* x, const float* norm_f,
              const float* norm_e, const float* norm_h, float eps, int64_t M, int64_t K, int8_t* xq,
              float* dx, int32_t* xs) {
    const char* fn = "wq_mtp_in";
    REQUIRE_PTR(emb);
    REQUIRE_PTR(x);
    REQUIRE_PTR(norm_f);
    REQUIRE_PTR(norm_e);
    REQUIRE_PTR(norm_h);
    REQUIRE_PTR(xq);
    REQUIRE_PTR(dx);
    REQUIRE_PTR(xs);
    if (M < 1 || M > (int64_t(1) << 29))
        return fail(WQ_ESHAPE, "%s: M = %lld out of range", fn, (long long)M);
    if (K < 128 || K % 128 != 0 || K > (int64_t(1) << 24))
        return fail(WQ_ESHAPE, "%s: K = %lld must be a positive multiple of 128", fn, (long long)K);
    if (!(eps >= 0.0f)) return fail(WQ_EINVAL, "%s: eps must be >= 0", fn);
    REQUIRE_ALIGN(emb, 16);
    REQUIRE_ALIGN(x, 16);
    REQUIRE_ALIGN(norm_f, 16);
    REQUIRE_ALIGN(norm_e, 16);
    REQUIRE_ALIGN(norm_h, 16);
    REQUIRE_ALIGN(xq, 16);
    REQUIRE_ALIGN(dx, 4);
    REQUIRE_ALIGN(xs, 4);
    wq::MtpInArgs a{emb, x, norm_f, norm_e, norm_h, eps, M, K, xq, dx, xs};
    return hip_status(wq::launch_mtp_in(a, static_cast<hipStream_t>(stream)), fn);
}

int wq_attn_combine(void* stream, const float* part, int64_t M, int64_t H, int64_t D, int64_t nch,
                    int64_t pos, const float* gate, int64_t gate_stride, int8_t* xq, float* dx,
                    int32_t* xs, const wq_params* params) {
    const char* fn = "wq_attn_combine";
    REQUIRE_PTR(part);
    REQUIRE_PTR(xq);
    REQUIRE_PTR(dx);
    REQUIRE_PTR(xs);
    if (D != 64 && D != 128 && D != 256)
        return fail(WQ_ESHAPE, "%s: head dim D = %lld (64, 128 or 256)", fn, (long long)D);
    if (M < 1 || M > 64) return fail(WQ_ESHAPE, "%s: M = %lld tokens (1..64)", fn, (long long)M);
    if (H < 1 || H > 1024) return fail(WQ_ESHAPE, "%s: H = %lld heads (1..1024)", fn, (long long)H);
    if (nch < 1 || nch > wq::kCombineMaxChunks)
        return fail(WQ_ESHAPE, "%s: nch = %lld chunks (1..%d)", fn, (long long)nch,
                    wq::kCombineMaxChunks);
    if (pos < 0 || pos + M - 1 >= 32 * nch)
        return fail(WQ_ESHAPE, "%s: positions 0..%lld exceed the %lld-position context", fn,
                    (long long)(pos + M - 1), (long long)(32 * nch));
    if (gate && gate_stride < 2 * H * D)
        return fail(WQ_ESHAPE, "%s: gate_stride = %lld < 2 H D = %lld", fn, (long long)gate_stride,
                    (long long)(2 * H * D));
    REQUIRE_ALIGN(part, 4);
    if (gate) REQUIRE_ALIGN(gate, 4);
    REQUIRE_ALIGN(xq, 16);
    REQUIRE_ALIGN(dx, 4);
    REQUIRE_ALIGN(xs, 4);
    if (params) REQUIRE_ALIGN(params, 4);
    wq::AttnCombineArgs a{part, M, H, D, nch, pos, reinterpret_cast<const uint32_t*>(params), gate,
                          gate_stride, xq, dx, xs};
    return hip_status(wq::launch_attn_combine(a, static_cast<hipStream_t>(stream)), fn);
}

size_t wq_lm_head_workspace_bytes(void) { return wq::kArgmaxWorkspaceBytes; }

int wq_workspace_clear(void* stream, void* workspace, size_t bytes) {
    const char* fn = "wq_workspace_clear";
    REQUIRE_PTR(workspace);
    if (bytes == 0) return ok();
    return hip_status(wq::launch_fill_zero(workspace, bytes, static_cast<hipStream_t>(stream)), fn);
}

namespace {

int lm_head_check(const char* fn, const uint32_t* wq, const uint32_t* ws, int64_t V, int64_t K,
                  int32_t G, const int8_t* xq, const float* dx, const int32_t* xs, int64_t M,
                  int32_t GA, float* logits, uint32_t* tok_out) {
    int rc = check_linear(fn, wq, ws, V, K, G, xq, dx, xs, M, GA, WQ_MODE_STORE, logits, false);
    if (rc) return rc;
    rc = check_gemv_shape(fn, M, K);
    if (rc) return rc;
    REQUIRE_PTR(tok_out);
    REQUIRE_ALIGN(tok_out, 4);
    if (V > (int64_t)0xFFFFFFFEll) return fail(WQ_ESHAPE, "%s: V = %lld out of range", fn, (long long)V);
    return WQ_OK;
}

int lm_head_launch(const char* fn, void* stream, const uint32_t* wq, const uint32_t* ws, int64_t V,
                   int64_t K, int32_t G, const int8_t* xq, const float* dx, const int32_t* xs,
                   int64_t M, int32_t GA, const uint32_t* ids, float* logits, uint32_t* tok_out,
                   void* workspace) {
    auto a = make_args(wq, ws, V, K, G, xq, dx, xs, M, GA, WQ_MODE_STORE, logits, nullptr);
    wq::ArgmaxArgs am{};
    am.ids = ids;
    am.tok_out = tok_out;
    am.keys = static_cast<unsigned long long*>(workspace);
    am.ticket = reinterpret_cast<unsigned int*>(static_cast<unsigned char*>(workspace) + wq::kArgmaxKeyBytes);
    return hip_status(wq::launch_lm_head_argmax(a, am, static_cast<hipStream_t>(stream)), fn);
}

}  // namespace

int wq_lm_head_argmax(void* stream, const uint32_t* wq, const uint32_t* ws, int64_t V, int64_t K,
                      int32_t G, const int8_t* xq, const float* dx, const int32_t* xs, int64_t M,
                      int32_t GA, const uint32_t* ids, float* logits, uint32_t* tok_out,
                      void* workspace, size_t workspace_bytes) {
    const char* fn = "wq_lm_head_argmax";
    int rc = lm_head_check(fn, wq, ws, V, K, G, xq, dx, xs, M, GA, logits, tok_out);
    if (rc) return rc;
    if (!workspace || workspace_bytes < wq::kArgmaxWorkspaceBytes)
        return fail(WQ_EWORKSPACE, "%s: workspace of %zu bytes required", fn,
                    (size_t)wq::kArgmaxWorkspaceBytes);
    REQUIRE_ALIGN(workspace, 8);
    return lm_head_launch(fn, stream, wq, ws, V, K, G, xq, dx, xs, M, GA, ids, logits, tok_out, workspace);
}

int wq_lm_head_argmax_noalloc(void* stream, const uint32_t* wq, const uint32_t* ws, int64_t V,
                              int64_t K, int32_t G, const int8_t* xq, const float* dx,
                              const int32_t* xs, int64_t M, int32_t GA, const uint32_t* ids,
                              float* logits, uint32_t* tok_out) {
    const char* fn = "wq_lm_head_argmax_noalloc";
    int rc = lm_head_check(fn, wq, ws, V, K, G, xq, dx, xs, M, GA, logits, tok_out);
    if (rc) return rc;
    // each of the scratch's kArgmaxSlots slots holds one running key per token
    if (M > wq::kArgmaxSlotWords)
        return fail(WQ_ESHAPE, "%s: M = %lld tokens exceeds the %d the scratch holds", fn, (long long)M,
                    wq::kArgmaxSlotWords);
    void* p = nullptr;
    hipError_t e = scratch_ptr(&p);
    if (e != hipSuccess) return hip_status(e, "wq_lm_head_argmax_noalloc: scratch address");
    return lm_head_launch(fn, stream, wq, ws, V, K, G, xq, dx, xs, M, GA, ids, logits, tok_out, p);
}

int wq_lm_head_noalloc_reset(void* stream) {
    const char* fn = "wq_lm_head_noalloc_reset";
    void* p = nullptr;
    hipError_t e = scratch_ptr(&p);
    if (e != hipSuccess) return hip_status(e, "wq_lm_head_noalloc_reset: scratch address");
    return hip_status(wq::launch_fill_zero(p, wq::kArgmaxWorkspaceBytes, static_cast<hipStream_t>(stream)), fn);
}

}  // extern "C"
