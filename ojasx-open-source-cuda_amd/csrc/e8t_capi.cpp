// e8t_capi.cpp -- extern "C" entry points of libojasx_e8t.so (declared in
// include/ojasx_e8t.h).  Validates arguments the way the reference's native
// binding does (ojasx_math_bindings.cpp:17-34, 414-433), checks the device,
// picks a kernel and enqueues it on the caller's stream.  The only mutable state
// is a per-device arch cache and a thread-local error message.  Nothing here
// allocates device memory: the prefill GEMM's K-split scratch is the caller's
// workspace argument (size from ojx_gemm_workspace_bytes).

#include <hip/hip_runtime.h>

#include <atomic>
#include <cstdarg>
#include <cstdio>
#include <cstddef>
#include <cstring>

#include "../../include/ojasx_e8t.h"
#include "e8t_device.h"
#include "e8t_internal.h"

namespace {

thread_local char g_last_error[512] = "";

int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int fail(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
    va_end(ap);
    return code;
}

int hip_fail(hipError_t e, const char* what) {
    return fail(OJX_EHIP, "%s: %s", what, hipGetErrorString(e));
}

constexpr int kMaxDevices = 64;
std::atomic<int> g_arch_ok[kMaxDevices];  // 0 unknown, 1 gfx950, 2 other

int check_device() {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
    if (dev < 0 || dev >= kMaxDevices) return fail(OJX_EDEVICE, "device index %d out of range", dev);
    int st = g_arch_ok[dev].load(std::memory_order_relaxed);
    if (st == 0) {
        hipDeviceProp_t prop;
        e = hipGetDeviceProperties(&prop, dev);
        if (e != hipSuccess) return hip_fail(e, "hipGetDeviceProperties");
        st = (std::strncmp(prop.gcnArchName, "gfx950", 6) == 0) ? 1 : 2;
        g_arch_ok[dev].store(st, std::memory_order_relaxed);
        if (st == 2)
            return fail(OJX_EDEVICE, "device %d is %s; this library is built for gfx950 only", dev,
                        prop.gcnArchName);
    }
    if (st == 2) return fail(OJX_EDEVICE, "device %d is not gfx950", dev);
    return OJX_OK;
}

bool valid_dtype(int dt) { return dt == OJX_F32 || dt == OJX_F16 || dt == OJX_BF16; }

int check_gs(int64_t gs) {
    if (gs <= 0 || gs % 16 != 0)
        return fail(OJX_ELAYOUT, "group_size must be a positive multiple of 16 (got %lld)",
                    (long long)gs);
    return OJX_OK;
}

int done(hipError_t e, const char* what) {
    if (e != hipSuccess) return hip_fail(e, what);
    g_last_error[0] = '\0';
    return OJX_OK;
}

}  // namespace

namespace ojx {
int api_fail(int code, const char* msg) { return fail(code, "%s", msg); }
}  // namespace ojx

// The prefill MFMA GEMM with its tile configuration and K split.  The split's fp32 partial
// sums live in the caller's workspace; a workspace smaller than the plan's (or none) lowers
// the split count to what fits, down to the unsplit kernel.
// bwd: the backward dX (output [M, K], reduction over N).
static hipError_t launch_mfma(const void* x, const uint8_t* packed, const uint16_t* scales,
                              const void* bias, void* y, int64_t M, int64_t N, int64_t K,
                              int64_t gs, int dtype, hipStream_t s, int fmt, bool bwd,
                              void* ws, size_t ws_bytes, const ojx::LoraEp& lora = ojx::LoraEp{}) {
    const int64_t out_cols = bwd ? K : N, red = bwd ? N : K;
    ojx::GemmChoice c = ojx::gemm_mfma_choice(M, out_cols, red, bwd);
    const size_t per = (size_t)ojx::split_stride(M, out_cols) * sizeof(float);
    const int64_t fit = ws ? (int64_t)(ws_bytes / per) : 0;
    if (c.splits > fit) c.splits = fit < 2 ? 1 : (int)fit;
    float* part = c.splits > 1 ? static_cast<float*>(ws) : nullptr;
    return ojx::launch_gemm_mfma(x, packed, scales, bias, y, part, c, M, N, K, dtype, s, gs, fmt,
                                 bwd, lora);
}

// Workspace pointer contract shared by the GEMM entry points.
static int check_workspace(const void* ws, size_t ws_bytes) {
    if (ws_bytes > 0 && !ws) return fail(OJX_EINVAL, "workspace_bytes %zu with a null workspace",
                                         ws_bytes);
    if ((uintptr_t)ws & 15u) return fail(OJX_ELAYOUT, "workspace must be 16-byte aligned");
    return OJX_OK;
}

// Group-size rule of each format's fused ops: ternary a multiple of 16 (the native op's
// packing unit, ojasx_math_bindings.cpp:17-34), 2-bit a multiple of 4 (bindings.cpp:285),
// 1-bit a multiple of 8 (the Root-E8 packer's unit).
static int check_gs_multiple(int64_t gs, int64_t unit) {
    if (gs <= 0 || gs % unit != 0)
        return fail(OJX_ELAYOUT, "group_size must be a positive multiple of %lld (got %lld)",
                    (long long)unit, (long long)gs);
    return OJX_OK;
}

static int64_t gs_unit(int fmt) {
    return fmt == ojx::kFmtTernary ? 16 : fmt == ojx::kFmt2Bit ? 4 : 8;
}

// a: x (forward) or grad_y (backward); out: y or grad_x; (M, N, K) the forward's shape.
static int check_fmt_args(int fmt, const void* a, const uint8_t* packed, const uint16_t* scales,
                          const void* out, int64_t M, int64_t out_cols, int64_t red, int64_t gs,
                          int dtype) {
    if (M < 0 || out_cols < 0 || red < 0)
        return fail(OJX_EINVAL, "negative size M=%lld, %lld x %lld", (long long)M,
                    (long long)out_cols, (long long)red);
    if (!valid_dtype(dtype)) return fail(OJX_EDTYPE, "unknown dtype code %d", dtype);
    if (int r = check_gs_multiple(gs, gs_unit(fmt))) return r;
    if (M > 0 && out_cols > 0) {
        if (!out) return fail(OJX_EINVAL, "null output pointer");
        if (red > 0 && (!a || !packed || !scales)) return fail(OJX_EINVAL, "null input pointer");
    }
    return OJX_OK;
}

// Kernel family of a forward / backward launch (the dispatch below).  Pointer alignment
// takes part in it; the workspace query passes null pointers (aligned).
enum Route { kRouteGemvTile, kRouteGemv2m, kRouteGemv, kRouteGemv2, kRouteMfma, kRouteGeneric };


static Route route_fwd(int fmt, const void* x, const uint8_t* packed, const uint16_t* scales,
                       const void* y, int64_t M, int64_t N, int64_t K, int64_t gs, int dtype) {
    if (fmt == ojx::kFmtTernary) {
        // layers too small to stream (per-linear decode launches), M <= 4: staged tiles
        if ((N + 15) / 16 < 1024 &&
            ojx::gemv_tile_supported(x, packed, scales, y, M, N, K, gs, dtype))
            return kRouteGemvTile;
        // 4 < M <= 16 on a layer too small for the streaming mask kernel (< 1024 row tiles):
        // one 16-row tile per workgroup, K split over its waves, weights in the B operand
        if (M > 4 && (N + 15) / 16 < 1024 &&
            ojx::gemv2m_supported(x, packed, scales, y, M, N, K, gs, dtype, fmt))
            return kRouteGemv2m;
        // group sizes 16 and 64 at M <= 16: the B-operand GEMV at every layer size
        if (gs != 32 && M <= 16 &&
            ojx::gemv2m_supported(x, packed, scales, y, M, N, K, gs, dtype, fmt))
            return kRouteGemv2m;
        if (K > 0 && ojx::gemv_supported(x, packed, scales, y, M, N, K, gs, dtype))
            return kRouteGemv;
        if (M > 16 && ojx::gemm_mfma_supported(x, packed, scales, M, N, K, gs, dtype, fmt))
            return kRouteMfma;
        return kRouteGeneric;
    }
    if (ojx::gemv2_supported(x, packed, scales, y, M, N, K, gs, dtype, fmt))
        return kRouteGemv2;
    if (ojx::gemv2m_supported(x, packed, scales, y, M, N, K, gs, dtype, fmt)) return kRouteGemv2m;
    if (ojx::gemm_mfma_supported(x, packed, scales, M, N, K, gs, dtype, fmt)) return kRouteMfma;
    return kRouteGeneric;
}

static Route route_bwd(int fmt, const void* gy, const uint8_t* packed, const uint16_t* scales,
                       int64_t M, int64_t N, int64_t K, int64_t gs, int dtype) {
    if (N > 0 && ojx::gemm_mfma_supported(gy, packed, scales, M, N, K, gs, dtype, fmt, true))
        return kRouteMfma;
    return kRouteGeneric;
}

static const char* fmt_name(int fmt) {
    return fmt == ojx::kFmtTernary ? "e8t" : fmt == ojx::kFmt2Bit ? "e8" : "e8r";
}

// Forward of every format: y[M, N] = x . Wdeq^T (+ bias).
static int gemm_fwd(int fmt, const void* x, const uint8_t* packed, const uint16_t* scales,
                    const void* bias, void* y, int64_t M, int64_t N, int64_t K, int64_t gs,
                    int dtype, void* ws, size_t ws_bytes, void* stream,
                    const ojx::LoraEp& lora = ojx::LoraEp{}, const void* lora_a_in = nullptr,
                    float lora_scaling = 0.f) {
    if (int r = check_fmt_args(fmt, x, packed, scales, y, M, N, K, gs, dtype)) return r;
    if (int r = check_workspace(ws, ws_bytes)) return r;
    if (M == 0 || N == 0) return OJX_OK;
    if (int r = check_device()) return r;
    hipStream_t s = (hipStream_t)stream;
    hipError_t e = hipSuccess;
    switch (route_fwd(fmt, x, packed, scales, y, M, N, K, gs, dtype)) {
    case kRouteGemvTile: {
        ojx::GemvLaunch a{};
        ojx::GemvJob& j = a.inl[0];
        j.x = x; j.packed = packed; j.scales = scales; j.bias = bias; j.y = y;
        j.N = N; j.K = K; j.y_col = 0; j.y_ld = N; j.wg_begin = 0;
        j.lora_u = lora.u; j.lora_b = lora.b; j.lora_r = lora.r; j.lora_ldu = lora.ldu;
        if (lora_a_in) {  // u formed inside the launch (gemm_fwd_lora checked the plan)
            j.lora_a = lora_a_in;
            j.lora_scaling = lora_scaling;
            a.lora_inline = 1;
        }
        a.njobs = 1;
        a.M = (int)M;
        e = ojx::launch_gemv_tile(a, (N + 15) / 16, K, dtype, s, gs);
        break;
    }
    case kRouteGemv2m:
        e = ojx::launch_gemv2m(x, packed, scales, bias, y, M, N, K, gs, dtype, s, fmt, lora);
        break;
    case kRouteGemv2:
        e = ojx::launch_gemv2(x, packed, scales, bias, y, M, N, K, gs, dtype, s, lora, fmt);
        break;
    case kRouteGemv: {
        ojx::GemvLaunch a{};
        ojx::GemvJob& j = a.inl[0];
        j.x = x; j.packed = packed; j.scales = scales; j.bias = bias; j.y = y;
        j.N = N; j.K = K; j.y_col = 0; j.y_ld = N; j.wg_begin = 0;
        j.lora_u = lora.u; j.lora_b = lora.b; j.lora_r = lora.r; j.lora_ldu = lora.ldu;
        a.njobs = 1;
        a.M = (int)M;
        const ojx::GemvPlan plan = ojx::gemv_pick((N + 15) / 16, M);
        e = ojx::launch_gemv(a, plan, ojx::gemv_wgs_for(N, plan), dtype, s);
        break;
    }
    case kRouteMfma:
        e = launch_mfma(x, packed, scales, bias, y, M, N, K, gs, dtype, s, fmt, false, ws,
                        ws_bytes, lora);
        break;
    case kRouteGeneric:
        e = ojx::launch_gemm_generic_fwd(x, packed, scales, bias, y, M, N, K, gs, dtype, s, fmt,
                                         lora);
        break;
    }
    if (e != hipSuccess) return fail(OJX_EHIP, "%s gemm_fwd launch: %s", fmt_name(fmt),
                                     hipGetErrorString(e));
    g_last_error[0] = '\0';
    return OJX_OK;
}

// Forward with a LoRA adapter: u = scaling * (x @ A) into the caller's lora_u, then the
// format's forward with u @ B added in its output epilogue.  The staged-tile GEMV with one
// round per wave forms u itself (rank 8): one launch, lora_u left untouched.
static int gemm_fwd_lora(int fmt, const void* x, const uint8_t* packed, const uint16_t* scales,
                         const void* bias, const void* lora_a, const void* lora_b, int64_t rank,
                         float scaling, float* lora_u, void* y, int64_t M, int64_t N, int64_t K,
                         int64_t gs, int dtype, void* ws, size_t ws_bytes, void* stream) {
    if (rank < 1 || rank > ojx::kLoraMaxRank)
        return fail(OJX_ELAYOUT, "LoRA rank must be in 1..%lld (got %lld)",
                    (long long)ojx::kLoraMaxRank, (long long)rank);
    if (M > 0 && N > 0 && (!lora_a || !lora_b || !lora_u))
        return fail(OJX_EINVAL, "null LoRA pointer");
    // every check of the forward runs before the down-projection is enqueued: a refused call
    // launches nothing
    if (((uintptr_t)lora_u & 3u) || ((uintptr_t)lora_a & 1u) || ((uintptr_t)lora_b & 1u))
        return fail(OJX_ELAYOUT, "misaligned LoRA operand (lora_u 4-byte, A and B 2-byte)");
    if (int r = check_fmt_args(fmt, x, packed, scales, y, M, N, K, gs, dtype)) return r;
    if (int r = check_workspace(ws, ws_bytes)) return r;
    if (M == 0 || N == 0) return OJX_OK;
    if (int r = check_device()) return r;
    const bool inline_u =
        route_fwd(fmt, x, packed, scales, y, M, N, K, gs, dtype) == kRouteGemvTile &&
        ojx::gemv_tile_lora_inline_ok(M, N, K, rank, lora_a);
    if (!inline_u) {
        const hipError_t e = ojx::launch_lora_down(x, lora_a, M, K, rank, scaling, dtype,
                                                   lora_u, rank, (hipStream_t)stream);
        if (e != hipSuccess) return fail(OJX_EHIP, "lora_down launch: %s", hipGetErrorString(e));
    }
    return gemm_fwd(fmt, x, packed, scales, bias, y, M, N, K, gs, dtype, ws, ws_bytes, stream,
                    ojx::LoraEp{lora_u, lora_b, rank, rank, N}, inline_u ? lora_a : nullptr,
                    scaling);
}

// Backward dX of every format: grad_x[M, K] = grad_y[M, N] . Wdeq[N, K].
static int gemm_bwd(int fmt, const void* grad_y, const uint8_t* packed, const uint16_t* scales,
                    void* grad_x, int64_t M, int64_t N, int64_t K, int64_t gs, int dtype,
                    void* ws, size_t ws_bytes, void* stream) {
    if (int r = check_fmt_args(fmt, grad_y, packed, scales, grad_x, M, K, N, gs, dtype)) return r;
    if (int r = check_workspace(ws, ws_bytes)) return r;
    if (M == 0 || K == 0) return OJX_OK;
    if (int r = check_device()) return r;
    hipStream_t s = (hipStream_t)stream;
    hipError_t e;
    if (route_bwd(fmt, grad_y, packed, scales, M, N, K, gs, dtype) == kRouteMfma)
        e = launch_mfma(grad_y, packed, scales, nullptr, grad_x, M, N, K, gs, dtype, s, fmt, true,
                        ws, ws_bytes);
    else
        e = ojx::launch_gemm_generic_bwd(grad_y, packed, scales, grad_x, M, N, K, gs, dtype, s,
                                         fmt);
    if (e != hipSuccess) return fail(OJX_EHIP, "%s gemm_bwd_dx launch: %s", fmt_name(fmt),
                                     hipGetErrorString(e));
    g_last_error[0] = '\0';
    return OJX_OK;
}

// Workspace bytes of a fused forward (bwd 0) or backward dX (bwd 1) launch.
static int workspace_bytes(int fmt, int bwd, int64_t M, int64_t N, int64_t K, int64_t gs,
                           int dtype, size_t* bytes) {
    if (!bytes) return fail(OJX_EINVAL, "null result pointer");
    *bytes = 0;
    if (fmt != ojx::kFmtTernary && fmt != ojx::kFmt2Bit && fmt != ojx::kFmtRoot)
        return fail(OJX_EINVAL, "unknown format code %d", fmt);
    if (M < 0 || N < 0 || K < 0) return fail(OJX_EINVAL, "negative size M=%lld N=%lld K=%lld",
                                             (long long)M, (long long)N, (long long)K);
    if (!valid_dtype(dtype)) return fail(OJX_EDTYPE, "unknown dtype code %d", dtype);
    if (int r = check_gs_multiple(gs, gs_unit(fmt))) return r;
    if (M == 0 || N == 0 || K == 0) return OJX_OK;
    const Route r = bwd ? route_bwd(fmt, nullptr, nullptr, nullptr, M, N, K, gs, dtype)
                        : route_fwd(fmt, nullptr, nullptr, nullptr, nullptr, M, N, K, gs, dtype);
    if (r == kRouteMfma) {
        const int64_t out_cols = bwd ? K : N, red = bwd ? N : K;
        *bytes = ojx::gemm_split_bytes(ojx::gemm_mfma_choice(M, out_cols, red, bwd != 0), M,
                                       out_cols);
    }
    g_last_error[0] = '\0';
    return OJX_OK;
}

extern "C" {

__attribute__((visibility("default"))) int ojx_e8t_version(void) { return 20000; }

__attribute__((visibility("default"))) const char* ojx_e8t_last_error(void) {
    return g_last_error;
}

__attribute__((visibility("default"))) int ojx_e8t_encode(const void* w, int w_dtype,
                                                          int64_t numel, int64_t gs,
                                                          uint8_t* packed, uint16_t* scales,
                                                          void* stream) {
    if (numel < 0) return fail(OJX_EINVAL, "negative numel %lld", (long long)numel);
    if (!valid_dtype(w_dtype)) return fail(OJX_EDTYPE, "unknown dtype code %d", w_dtype);
    if (int r = check_gs(gs)) return r;
    if (numel == 0) return OJX_OK;
    if (!w || !packed || !scales) return fail(OJX_EINVAL, "null pointer");
    if (int r = check_device()) return r;
    return done(ojx::launch_encode(w, w_dtype, numel, gs, packed, scales, (hipStream_t)stream),
                "e8t encode launch");
}

__attribute__((visibility("default"))) int ojx_e8t_decode(const uint8_t* packed,
                                                          const uint16_t* scales, int64_t numel,
                                                          int64_t gs, int out_dtype, void* out,
                                                          void* stream) {
    if (numel < 0) return fail(OJX_EINVAL, "negative numel %lld", (long long)numel);
    if (!valid_dtype(out_dtype)) return fail(OJX_EDTYPE, "unknown dtype code %d", out_dtype);
    if (int r = check_gs(gs)) return r;
    if (numel == 0) return OJX_OK;
    if (!packed || !scales || !out) return fail(OJX_EINVAL, "null pointer");
    if (int r = check_device()) return r;
    return done(ojx::launch_decode(packed, scales, numel, gs, out_dtype, out, (hipStream_t)stream),
                "e8t decode launch");
}

static_assert(sizeof(ojx_e8t_gemv_job) == sizeof(ojx::GemvJob), "job layout");
static_assert(offsetof(ojx_e8t_gemv_job, wg_begin) == offsetof(ojx::GemvJob, wg_begin),
              "job layout");

// The adapters' down-projections u = scaling * x @ A of a job table, before its GEMV:
// consecutive adapter jobs on the same activations (same x, same K) share a launch.
static int lora_downs(const ojx_e8t_gemv_job* jobs, int njobs, const void* x, int64_t M,
                      int dtype, void* stream) {
    for (int i = 0; i < njobs;) {
        if (jobs[i].lora_r <= 0) { ++i; continue; }
        const void* xi = jobs[i].x ? jobs[i].x : x;
        const int64_t Ki = jobs[i].K;
        ojx::LoraDown items[ojx::kLoraDownItems];
        int n = 0;
        for (; i < njobs && n < ojx::kLoraDownItems; ++i) {
            const ojx_e8t_gemv_job& j = jobs[i];
            if (j.lora_r <= 0) continue;
            if ((j.x ? j.x : x) != xi || j.K != Ki) break;
            items[n++] = ojx::LoraDown{j.lora_a, const_cast<float*>(j.lora_u), j.lora_r,
                                       j.lora_ldu ? j.lora_ldu : j.lora_r, j.lora_scaling};
        }
        const hipError_t e = ojx::launch_lora_down(xi, M, Ki, dtype, items, n,
                                                   (hipStream_t)stream);
        if (e != hipSuccess) return fail(OJX_EHIP, "lora_down launch: %s", hipGetErrorString(e));
    }
    return OJX_OK;
}

static int plan_jobs(ojx_e8t_gemv_job* jobs, int njobs, int64_t M, int dtype, int64_t* grid,
                     ojx::GemvPlan* plan, bool fill) {
    if (njobs <= 0 || !jobs) return fail(OJX_EINVAL, "empty job list");
    if (dtype != OJX_BF16 && dtype != OJX_F16)
        return fail(OJX_EDTYPE, "grouped GEMV takes F16 or BF16 activations (got %d)", dtype);
    if (M < 1 || M > 16) return fail(OJX_ELAYOUT, "grouped GEMV needs 1 <= M <= 16 (got %lld)",
                                     (long long)M);
    int64_t tiles = 0, kmax = 0;
    bool tile_ok = M <= 4;
    for (int i = 0; i < njobs; ++i) {
        const ojx_e8t_gemv_job& j = jobs[i];
        kmax = j.K > kmax ? j.K : kmax;
        tile_ok = tile_ok && j.K % 1024 == 0 && ((uintptr_t)j.packed & 15u) == 0 &&
                  ((uintptr_t)j.scales & 15u) == 0 && (j.N + 16) * (j.K * 3 / 16) < (1ll << 31) &&
                  M * j.K * 2 < (1ll << 31);
        if (j.N < 1 || j.K < 256 || j.K % 256 != 0)
            return fail(OJX_ELAYOUT, "job %d: needs N >= 1 and K %% 256 == 0 (N=%lld K=%lld)", i,
                        (long long)j.N, (long long)j.K);
        if (!ojx::gemv_shape_ok(j.N, j.K))
            return fail(OJX_ELAYOUT, "job %d: layer too large for 32-bit offsets", i);
        if (!j.packed || !j.scales) return fail(OJX_EINVAL, "job %d: null weight pointer", i);
        if (((uintptr_t)j.packed & 3u) || ((uintptr_t)j.scales & 3u) || ((uintptr_t)j.x & 15u) ||
            ((uintptr_t)j.y & 1u) || ((uintptr_t)j.bias & 1u))
            return fail(OJX_ELAYOUT, "job %d: misaligned pointer", i);
        if (j.lora_r < 0 || j.lora_r > ojx::kLoraMaxRank)
            return fail(OJX_ELAYOUT, "job %d: LoRA rank must be in 0..%lld", i,
                        (long long)ojx::kLoraMaxRank);
        if (j.lora_r > 0 && (!j.lora_u || !j.lora_b || !j.lora_a || ((uintptr_t)j.lora_u & 3u) ||
                             ((uintptr_t)j.lora_b & 1u) || ((uintptr_t)j.lora_a & 1u) ||
                             (j.lora_ldu != 0 && j.lora_ldu < j.lora_r)))
            return fail(OJX_EINVAL, "job %d: bad LoRA operands", i);
        const int64_t ld = j.y_ld ? j.y_ld : j.N;
        if (j.y_col < 0 || ld < j.y_col + j.N)
            return fail(OJX_ELAYOUT, "job %d: y_ld %lld < y_col %lld + N %lld", i, (long long)ld,
                        (long long)j.y_col, (long long)j.N);
        tiles += (j.N + 15) / 16;
    }
    *plan = ojx::gemv_pick_grouped(tiles, M, kmax, tile_ok);
    int64_t wg = 0;
    for (int i = 0; i < njobs; ++i) {
        if (fill) {
            jobs[i].wg_begin = wg;
            if (jobs[i].y_ld == 0) jobs[i].y_ld = jobs[i].N;
        } else if (jobs[i].wg_begin != wg || jobs[i].y_ld == 0) {
            return fail(OJX_EINVAL, "job %d: the job array was not planned for this M", i);
        }
        wg += ojx::gemv_wgs_for(jobs[i].N, *plan);
    }
    if (wg > 0x7FFFFFFF) return fail(OJX_ELAYOUT, "grouped GEMV grid too large");
    *grid = wg;
    return OJX_OK;
}

__attribute__((visibility("default"))) int ojx_e8t_gemv_grouped_plan(ojx_e8t_gemv_job* jobs,
                                                                     int njobs, int64_t M,
                                                                     int dtype, int64_t* grid) {
    int64_t g = 0;
    ojx::GemvPlan plan{};
    if (int r = plan_jobs(jobs, njobs, M, dtype, &g, &plan, true)) return r;
    if (grid) *grid = g;
    g_last_error[0] = '\0';
    return OJX_OK;
}

__attribute__((visibility("default"))) int ojx_e8t_gemv_grouped(
    const ojx_e8t_gemv_job* jobs, const ojx_e8t_gemv_job* jobs_dev, int njobs, const void* x,
    void* y, int64_t M, int dtype, void* stream) {
    int64_t grid = 0;
    ojx::GemvPlan plan{};
    if (int r = plan_jobs(const_cast<ojx_e8t_gemv_job*>(jobs), njobs, M, dtype, &grid, &plan,
                          false))
        return r;
    if (((uintptr_t)x & 15u) || ((uintptr_t)y & 1u))
        return fail(OJX_ELAYOUT, "misaligned default x / y");
    for (int i = 0; i < njobs; ++i) {
        if (!jobs[i].x && !x) return fail(OJX_EINVAL, "job %d has no activations", i);
        if (!jobs[i].y && !y) return fail(OJX_EINVAL, "job %d has no output", i);
    }
    if (!jobs_dev && njobs > ojx::kGemvInlineJobs)
        return fail(OJX_EINVAL, "more than %d jobs need a device job table",
                    ojx::kGemvInlineJobs);
    if (int r = check_device()) return r;
    ojx::GemvLaunch a{};
    if (!jobs_dev)
        for (int i = 0; i < njobs; ++i) std::memcpy(&a.inl[i], &jobs[i], sizeof(ojx::GemvJob));
    a.jobs = reinterpret_cast<const ojx::GemvJob*>(jobs_dev);
    a.x = x;
    a.y = y;
    a.njobs = njobs;
    a.M = (int)M;
    // staged-tile plans with one round per wave form the (rank-8) adapters' u themselves
    bool inline_u = plan.tile;
    for (int i = 0; i < njobs; ++i)
        if (jobs[i].lora_r > 0)
            inline_u = inline_u && ojx::gemv_lora_inline_ok(plan.U, plan.rt, plan.tpw,
                                                             jobs[i].lora_r, jobs[i].lora_a);
    a.lora_inline = inline_u ? 1 : 0;
    if (!inline_u)
        if (int r = lora_downs(jobs, njobs, x, M, dtype, stream)) return r;
    return done(ojx::launch_gemv(a, plan, grid, dtype, (hipStream_t)stream),
                "e8t grouped gemv launch");
}

// ------------------------------------------------------------------ grouped 2-bit / 1-bit GEMV

// Validates a 2-bit (fmt kFmt2Bit) or 1-bit (kFmtRoot) job table for batch M and group size
// gs, picks the plan and (fill) sets each job's first workgroup and default y_ld, or (!fill)
// checks that they were so set.
static int plan_jobs2(ojx_e8t_gemv_job* jobs, int njobs, int64_t M, int64_t gs, int dtype,
                      int64_t* grid, ojx::Gemv2Plan* plan, bool fill, int fmt) {
    const int64_t cdiv = fmt == ojx::kFmtRoot ? 8 : 4;  // weights per code byte
    if (njobs <= 0 || !jobs) return fail(OJX_EINVAL, "empty job list");
    if (dtype != OJX_BF16 && dtype != OJX_F16)
        return fail(OJX_EDTYPE, "grouped GEMV takes F16 or BF16 activations (got %d)", dtype);
    if (M < 1 || M > 16) return fail(OJX_ELAYOUT, "grouped GEMV needs 1 <= M <= 16 (got %lld)",
                                     (long long)M);
    if (gs != 8 && gs != 16 && gs != 32 && gs != 64)
        return fail(OJX_ELAYOUT, "grouped %s GEMV needs group size 8, 16, 32 or 64 (got %lld)",
                    fmt == ojx::kFmtRoot ? "1-bit" : "2-bit", (long long)gs);
    int64_t tiles = 0;
    bool k1024 = true;
    for (int i = 0; i < njobs; ++i) {
        const ojx_e8t_gemv_job& j = jobs[i];
        if (j.N < 1 || j.K < 256 || j.K % 256 != 0)
            return fail(OJX_ELAYOUT, "job %d: needs N >= 1 and K %% 256 == 0 (N=%lld K=%lld)", i,
                        (long long)j.N, (long long)j.K);
        if ((j.N + 32) * (j.K / cdiv) >= (1ll << 31) || (j.N + 32) * (j.K * 2 / gs) >= (1ll << 31) ||
            M * j.K * 2 >= (1ll << 31))
            return fail(OJX_ELAYOUT, "job %d: layer too large for 32-bit offsets", i);
        if (!j.packed || !j.scales) return fail(OJX_EINVAL, "job %d: null weight pointer", i);
        if (((uintptr_t)j.packed & 15u) || ((uintptr_t)j.scales & 15u) || ((uintptr_t)j.x & 15u) ||
            ((uintptr_t)j.y & 1u) || ((uintptr_t)j.bias & 1u))
            return fail(OJX_ELAYOUT, "job %d: misaligned pointer", i);
        if (j.lora_r < 0 || j.lora_r > ojx::kLoraMaxRank)
            return fail(OJX_ELAYOUT, "job %d: LoRA rank must be in 0..%lld", i,
                        (long long)ojx::kLoraMaxRank);
        if (j.lora_r > 0 && (!j.lora_u || !j.lora_b || !j.lora_a || ((uintptr_t)j.lora_u & 3u) ||
                             ((uintptr_t)j.lora_b & 1u) || ((uintptr_t)j.lora_a & 1u) ||
                             (j.lora_ldu != 0 && j.lora_ldu < j.lora_r)))
            return fail(OJX_EINVAL, "job %d: bad LoRA operands", i);
        const int64_t ld = j.y_ld ? j.y_ld : j.N;
        if (j.y_col < 0 || ld < j.y_col + j.N)
            return fail(OJX_ELAYOUT, "job %d: y_ld %lld < y_col %lld + N %lld", i, (long long)ld,
                        (long long)j.y_col, (long long)j.N);
        k1024 = k1024 && j.K % 1024 == 0;
        tiles += (j.N + 15) / 16;
    }
    *plan = ojx::gemv2_pick_grouped(tiles, M, k1024, fmt);
    int64_t wg = 0;
    for (int i = 0; i < njobs; ++i) {
        if (fill) {
            jobs[i].wg_begin = wg;
            if (jobs[i].y_ld == 0) jobs[i].y_ld = jobs[i].N;
        } else if (jobs[i].wg_begin != wg || jobs[i].y_ld == 0) {
            return fail(OJX_EINVAL, "job %d: the job array was not planned for this M", i);
        }
        wg += ojx::gemv2_wgs_for(jobs[i].N, *plan);
    }
    if (wg > 0x7FFFFFFF) return fail(OJX_ELAYOUT, "grouped GEMV grid too large");
    *grid = wg;
    return OJX_OK;
}

static int gemv2_grouped_plan(ojx_e8t_gemv_job* jobs, int njobs, int64_t M, int64_t gs,
                              int dtype, int64_t* grid, int fmt) {
    int64_t g = 0;
    ojx::Gemv2Plan plan{};
    if (int r = plan_jobs2(jobs, njobs, M, gs, dtype, &g, &plan, true, fmt)) return r;
    if (grid) *grid = g;
    g_last_error[0] = '\0';
    return OJX_OK;
}

static int gemv2_grouped(const ojx_e8t_gemv_job* jobs, const ojx_e8t_gemv_job* jobs_dev,
                         int njobs, const void* x, void* y, int64_t M, int64_t gs, int dtype,
                         void* stream, int fmt) {
    int64_t grid = 0;
    ojx::Gemv2Plan plan{};
    if (int r = plan_jobs2(const_cast<ojx_e8t_gemv_job*>(jobs), njobs, M, gs, dtype, &grid, &plan,
                           false, fmt))
        return r;
    if (((uintptr_t)x & 15u) || ((uintptr_t)y & 1u))
        return fail(OJX_ELAYOUT, "misaligned default x / y");
    for (int i = 0; i < njobs; ++i) {
        if (!jobs[i].x && !x) return fail(OJX_EINVAL, "job %d has no activations", i);
        if (!jobs[i].y && !y) return fail(OJX_EINVAL, "job %d has no output", i);
    }
    if (!jobs_dev && njobs > ojx::kGemvInlineJobs)
        return fail(OJX_EINVAL, "more than %d jobs need a device job table",
                    ojx::kGemvInlineJobs);
    if (int r = check_device()) return r;
    ojx::GemvLaunch a{};
    if (!jobs_dev)
        for (int i = 0; i < njobs; ++i) std::memcpy(&a.inl[i], &jobs[i], sizeof(ojx::GemvJob));
    a.jobs = reinterpret_cast<const ojx::GemvJob*>(jobs_dev);
    a.x = x;
    a.y = y;
    a.njobs = njobs;
    a.M = (int)M;
    if (int r = lora_downs(jobs, njobs, x, M, dtype, stream)) return r;
    return done(ojx::launch_gemv2_grouped(a, plan, grid, gs, dtype, fmt, (hipStream_t)stream),
                fmt == ojx::kFmtRoot ? "e8r grouped gemv launch" : "e8 grouped gemv launch");
}

__attribute__((visibility("default"))) int ojx_e8_gemv_grouped_plan(ojx_e8t_gemv_job* jobs,
                                                                    int njobs, int64_t M,
                                                                    int64_t gs, int dtype,
                                                                    int64_t* grid) {
    return gemv2_grouped_plan(jobs, njobs, M, gs, dtype, grid, ojx::kFmt2Bit);
}

__attribute__((visibility("default"))) int ojx_e8_gemv_grouped(
    const ojx_e8t_gemv_job* jobs, const ojx_e8t_gemv_job* jobs_dev, int njobs, const void* x,
    void* y, int64_t M, int64_t gs, int dtype, void* stream) {
    return gemv2_grouped(jobs, jobs_dev, njobs, x, y, M, gs, dtype, stream, ojx::kFmt2Bit);
}

__attribute__((visibility("default"))) int ojx_e8r_gemv_grouped_plan(ojx_e8t_gemv_job* jobs,
                                                                     int njobs, int64_t M,
                                                                     int64_t gs, int dtype,
                                                                     int64_t* grid) {
    return gemv2_grouped_plan(jobs, njobs, M, gs, dtype, grid, ojx::kFmtRoot);
}

__attribute__((visibility("default"))) int ojx_e8r_gemv_grouped(
    const ojx_e8t_gemv_job* jobs, const ojx_e8t_gemv_job* jobs_dev, int njobs, const void* x,
    void* y, int64_t M, int64_t gs, int dtype, void* stream) {
    return gemv2_grouped(jobs, jobs_dev, njobs, x, y, M, gs, dtype, stream, ojx::kFmtRoot);
}

// ------------------------------------------------------------------ 2-bit E8

__attribute__((visibility("default"))) int ojx_e8_encode(const void* w, int w_dtype,
                                                         int64_t numel, int64_t gs,
                                                         uint8_t* packed, uint16_t* scales,
                                                         void* stream) {
    if (numel < 0) return fail(OJX_EINVAL, "negative numel %lld", (long long)numel);
    if (!valid_dtype(w_dtype)) return fail(OJX_EDTYPE, "unknown dtype code %d", w_dtype);
    if (int r = check_gs_multiple(gs, 8)) return r;
    if (numel == 0) return OJX_OK;
    if (!w || !packed || !scales) return fail(OJX_EINVAL, "null pointer");
    if (int r = check_device()) return r;
    return done(ojx::launch_encode2(w, w_dtype, numel, gs, packed, scales, (hipStream_t)stream),
                "e8 encode launch");
}

__attribute__((visibility("default"))) int ojx_e8_decode(const uint8_t* packed,
                                                         const uint16_t* scales, int64_t numel,
                                                         int64_t gs, int out_dtype, void* out,
                                                         void* stream) {
    if (numel < 0) return fail(OJX_EINVAL, "negative numel %lld", (long long)numel);
    if (!valid_dtype(out_dtype)) return fail(OJX_EDTYPE, "unknown dtype code %d", out_dtype);
    if (int r = check_gs_multiple(gs, 8)) return r;
    if (numel == 0) return OJX_OK;
    if (!packed || !scales || !out) return fail(OJX_EINVAL, "null pointer");
    if (int r = check_device()) return r;
    return done(ojx::launch_decode2(packed, scales, numel, gs, out_dtype, out, (hipStream_t)stream),
                "e8 decode launch");
}

// ---------------------------------------------------------------- 1-bit Root E8

__attribute__((visibility("default"))) int ojx_e8r_encode(const void* w, int w_dtype,
                                                          int64_t numel, int64_t gs,
                                                          uint8_t* codes, uint16_t* scales,
                                                          void* stream) {
    if (numel < 0) return fail(OJX_EINVAL, "negative numel %lld", (long long)numel);
    if (!valid_dtype(w_dtype)) return fail(OJX_EDTYPE, "unknown dtype code %d", w_dtype);
    if (int r = check_gs_multiple(gs, 8)) return r;
    if (numel == 0) return OJX_OK;
    if (!w || !codes || !scales) return fail(OJX_EINVAL, "null pointer");
    if (int r = check_device()) return r;
    return done(ojx::launch_encode1(w, w_dtype, numel, gs, codes, scales, (hipStream_t)stream),
                "e8r encode launch");
}

__attribute__((visibility("default"))) int ojx_e8r_decode(const uint8_t* codes,
                                                          const uint16_t* scales, int64_t numel,
                                                          int64_t gs, int out_dtype, void* out,
                                                          void* stream) {
    if (numel < 0) return fail(OJX_EINVAL, "negative numel %lld", (long long)numel);
    if (!valid_dtype(out_dtype)) return fail(OJX_EDTYPE, "unknown dtype code %d", out_dtype);
    if (int r = check_gs_multiple(gs, 8)) return r;
    if (numel == 0) return OJX_OK;
    if (!codes || !scales || !out) return fail(OJX_EINVAL, "null pointer");
    if (int r = check_device()) return r;
    return done(ojx::launch_decode1(codes, scales, numel, gs, out_dtype, out, (hipStream_t)stream),
                "e8r decode launch");
}


__attribute__((visibility("default"))) int ojx_gemm_workspace_bytes(int fmt, int bwd, int64_t M,
                                                                    int64_t N, int64_t K,
                                                                    int64_t gs, int dtype,
                                                                    size_t* bytes) {
    return workspace_bytes(fmt, bwd, M, N, K, gs, dtype, bytes);
}

__attribute__((visibility("default"))) int ojx_e8t_gemm_fwd(
    const void* x, const uint8_t* packed, const uint16_t* scales, const void* bias, void* y,
    int64_t M, int64_t N, int64_t K, int64_t gs, int dtype, void* workspace,
    size_t workspace_bytes, void* stream) {
    return gemm_fwd(ojx::kFmtTernary, x, packed, scales, bias, y, M, N, K, gs, dtype, workspace,
                    workspace_bytes, stream);
}

__attribute__((visibility("default"))) int ojx_lora_down(const void* x, const void* lora_a,
                                                         int64_t M, int64_t K, int64_t rank,
                                                         float scaling, int dtype, float* u,
                                                         void* stream) {
    if (M < 0 || K < 0) return fail(OJX_EINVAL, "negative size M=%lld K=%lld", (long long)M,
                                    (long long)K);
    if (!valid_dtype(dtype)) return fail(OJX_EDTYPE, "unknown dtype code %d", dtype);
    if (rank < 1 || rank > ojx::kLoraMaxRank)
        return fail(OJX_ELAYOUT, "LoRA rank must be in 1..%lld (got %lld)",
                    (long long)ojx::kLoraMaxRank, (long long)rank);
    if (M == 0) return OJX_OK;
    if (!x || !lora_a || !u) return fail(OJX_EINVAL, "null pointer");
    if (int r = check_device()) return r;
    return done(ojx::launch_lora_down(x, lora_a, M, K, rank, scaling, dtype, u, rank,
                                      (hipStream_t)stream),
                "lora_down launch");
}

__attribute__((visibility("default"))) int ojx_e8t_gemm_fwd_lora(
    const void* x, const uint8_t* packed, const uint16_t* scales, const void* bias,
    const void* lora_a, const void* lora_b, int64_t rank, float scaling, float* lora_u, void* y,
    int64_t M, int64_t N, int64_t K, int64_t gs, int dtype, void* workspace,
    size_t workspace_bytes, void* stream) {
    return gemm_fwd_lora(ojx::kFmtTernary, x, packed, scales, bias, lora_a, lora_b, rank,
                         scaling, lora_u, y, M, N, K, gs, dtype, workspace, workspace_bytes,
                         stream);
}

__attribute__((visibility("default"))) int ojx_e8_gemm_fwd_lora(
    const void* x, const uint8_t* packed, const uint16_t* scales, const void* bias,
    const void* lora_a, const void* lora_b, int64_t rank, float scaling, float* lora_u, void* y,
    int64_t M, int64_t N, int64_t K, int64_t gs, int dtype, void* workspace,
    size_t workspace_bytes, void* stream) {
    return gemm_fwd_lora(ojx::kFmt2Bit, x, packed, scales, bias, lora_a, lora_b, rank, scaling,
                         lora_u, y, M, N, K, gs, dtype, workspace, workspace_bytes, stream);
}

__attribute__((visibility("default"))) int ojx_e8r_gemm_fwd_lora(
    const void* x, const uint8_t* codes, const uint16_t* scales, const void* bias,
    const void* lora_a, const void* lora_b, int64_t rank, float scaling, float* lora_u, void* y,
    int64_t M, int64_t N, int64_t K, int64_t gs, int dtype, void* workspace,
    size_t workspace_bytes, void* stream) {
    return gemm_fwd_lora(ojx::kFmtRoot, x, codes, scales, bias, lora_a, lora_b, rank, scaling,
                         lora_u, y, M, N, K, gs, dtype, workspace, workspace_bytes, stream);
}

__attribute__((visibility("default"))) int ojx_e8t_gemm_bwd_dx(
    const void* grad_y, const uint8_t* packed, const uint16_t* scales, void* grad_x, int64_t M,
    int64_t N, int64_t K, int64_t gs, int dtype, void* workspace, size_t workspace_bytes,
    void* stream) {
    return gemm_bwd(ojx::kFmtTernary, grad_y, packed, scales, grad_x, M, N, K, gs, dtype,
                    workspace, workspace_bytes, stream);
}

__attribute__((visibility("default"))) int ojx_e8_gemm_fwd(
    const void* x, const uint8_t* packed, const uint16_t* scales, const void* bias, void* y,
    int64_t M, int64_t N, int64_t K, int64_t gs, int dtype, void* workspace,
    size_t workspace_bytes, void* stream) {
    return gemm_fwd(ojx::kFmt2Bit, x, packed, scales, bias, y, M, N, K, gs, dtype, workspace,
                    workspace_bytes, stream);
}

__attribute__((visibility("default"))) int ojx_e8_gemm_bwd_dx(
    const void* grad_y, const uint8_t* packed, const uint16_t* scales, void* grad_x, int64_t M,
    int64_t N, int64_t K, int64_t gs, int dtype, void* workspace, size_t workspace_bytes,
    void* stream) {
    return gemm_bwd(ojx::kFmt2Bit, grad_y, packed, scales, grad_x, M, N, K, gs, dtype, workspace,
                    workspace_bytes, stream);
}

__attribute__((visibility("default"))) int ojx_e8r_gemm_fwd(
    const void* x, const uint8_t* codes, const uint16_t* scales, const void* bias, void* y,
    int64_t M, int64_t N, int64_t K, int64_t gs, int dtype, void* workspace,
    size_t workspace_bytes, void* stream) {
    return gemm_fwd(ojx::kFmtRoot, x, codes, scales, bias, y, M, N, K, gs, dtype, workspace,
                    workspace_bytes, stream);
}

__attribute__((visibility("default"))) int ojx_e8r_gemm_bwd_dx(
    const void* grad_y, const uint8_t* codes, const uint16_t* scales, void* grad_x, int64_t M,
    int64_t N, int64_t K, int64_t gs, int dtype, void* workspace, size_t workspace_bytes,
    void* stream) {
    return gemm_bwd(ojx::kFmtRoot, grad_y, codes, scales, grad_x, M, N, K, gs, dtype, workspace,
                    workspace_bytes, stream);
}

// ---------------------------------------------------------------- Hadamard rotation

__attribute__((visibility("default"))) int ojx_fwht32(const void* x, int dtype, int64_t numel,
                                                      void* y, void* stream) {
    if (!valid_dtype(dtype) && dtype != OJX_F64)
        return fail(OJX_EDTYPE, "unknown dtype code %d", dtype);
    if (numel < 0 || numel % 32 != 0)
        return fail(OJX_ELAYOUT, "numel %lld is not a multiple of 32", (long long)numel);
    if (numel == 0) return OJX_OK;
    if (!x || !y) return fail(OJX_EINVAL, "null pointer");
    if (((uintptr_t)x & 15u) || ((uintptr_t)y & 15u))
        return fail(OJX_ELAYOUT, "x and y must be 16-byte aligned");
    if (int r = check_device()) return r;
    return done(ojx::launch_fwht32(x, dtype, numel / 32, y, (hipStream_t)stream),
                "fwht32 launch");
}

// ---------------------------------------------------------------- QAT helpers

__attribute__((visibility("default"))) int ojx_e8_cs_project(const void* x, int f64,
                                                             int64_t nvec, void* out,
                                                             void* stream) {
    if (nvec < 0) return fail(OJX_EINVAL, "negative vector count %lld", (long long)nvec);
    if (nvec == 0) return OJX_OK;
    if (!x || !out) return fail(OJX_EINVAL, "null pointer");
    if (int r = check_device()) return r;
    return done(ojx::launch_cs_project(x, f64 != 0, nvec, out, (hipStream_t)stream),
                "e8 cs_project launch");
}

__attribute__((visibility("default"))) int ojx_e8_cs_project_dt(const void* x, int dtype,
                                                                int64_t nvec, void* out,
                                                                void* stream) {
    if (nvec < 0) return fail(OJX_EINVAL, "negative vector count %lld", (long long)nvec);
    if (dtype != OJX_F32 && dtype != OJX_F64 && dtype != OJX_F16 && dtype != OJX_BF16)
        return fail(OJX_EDTYPE, "unknown dtype code %d", dtype);
    if (nvec == 0) return OJX_OK;
    if (!x || !out) return fail(OJX_EINVAL, "null pointer");
    if (int r = check_device()) return r;
    return done(ojx::launch_cs_project_dt(x, dtype, nvec, out, (hipStream_t)stream),
                "e8 cs_project launch");
}

__attribute__((visibility("default"))) int ojx_e8_ste_quantize_dt(const void* w, int dtype,
                                                                  int64_t numel, void* out,
                                                                  void* stream) {
    if (numel < 0) return fail(OJX_EINVAL, "negative numel %lld", (long long)numel);
    if (dtype != OJX_F32 && dtype != OJX_F16 && dtype != OJX_BF16)
        return fail(OJX_EDTYPE, "ste_quantize takes F32, F16 or BF16 weights (got %d)", dtype);
    if (numel == 0) return OJX_OK;
    if (!w || !out) return fail(OJX_EINVAL, "null pointer");
    if (int r = check_device()) return r;
    return done(ojx::launch_ste_quantize_dt(w, dtype, numel, out, (hipStream_t)stream),
                "e8 ste_quantize launch");
}

__attribute__((visibility("default"))) int ojx_e8_ste_quantize(const float* w, int64_t numel,
                                                               float* out, void* stream) {
    if (numel < 0) return fail(OJX_EINVAL, "negative numel %lld", (long long)numel);
    if (numel == 0) return OJX_OK;
    if (!w || !out) return fail(OJX_EINVAL, "null pointer");
    if (int r = check_device()) return r;
    return done(ojx::launch_ste_quantize(w, numel, out, (hipStream_t)stream),
                "e8 ste_quantize launch");
}

}  // extern "C"
