// e8t_capi.cpp -- extern "C" entry points of libojasx_e8t.so (declared in
// include/ojasx_e8t.h).  Validates arguments the way the reference's native
// binding does (ojasx_math_bindings.cpp:17-34, 414-433), checks the device,
// picks a kernel and enqueues it on the caller's stream.  The only mutable state
// is a per-device arch cache, a thread-local error message and the prefill GEMM's
// K-split scratch (e8t_workspace.cpp: allocated only when a stream's buffer must
// grow, never during graph capture).

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

int check_gemm_args(const void* a, const uint8_t* packed, const uint16_t* scales, const void* out,
                    int64_t M, int64_t N, int64_t K, int64_t gs, int dtype) {
    if (M < 0 || N < 0 || K < 0) return fail(OJX_EINVAL, "negative size M=%lld N=%lld K=%lld",
                                             (long long)M, (long long)N, (long long)K);
    if (!valid_dtype(dtype)) return fail(OJX_EDTYPE, "unknown dtype code %d", dtype);
    if (int r = check_gs(gs)) return r;
    if (M > 0 && N > 0) {
        if (!out) return fail(OJX_EINVAL, "null output pointer");
        if (K > 0 && (!a || !packed || !scales)) return fail(OJX_EINVAL, "null input pointer");
    }
    return OJX_OK;
}

}  // namespace

extern "C" {

__attribute__((visibility("default"))) int ojx_e8t_version(void) { return 100; }

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

// The prefill MFMA GEMM with its tile configuration and K split; the split's fp32 partial
// sums live in the per-stream workspace (none while the stream is captured: unsplit).
// bwd: the backward dX (output [M, K], reduction over N).
static hipError_t launch_mfma(const void* x, const uint8_t* packed, const uint16_t* scales,
                              const void* bias, void* y, int64_t M, int64_t N, int64_t K,
                              int64_t gs, int dtype, hipStream_t s, int fmt, bool bwd = false) {
    const int64_t out_cols = bwd ? K : N, red = bwd ? N : K;
    ojx::GemmChoice c = ojx::gemm_mfma_choice(M, out_cols, red);
    float* part = nullptr;
    if (c.splits > 1) {
        part = static_cast<float*>(ojx::stream_workspace(
            s, (size_t)c.splits * (size_t)ojx::split_stride(M, out_cols) * sizeof(float)));
        if (!part) c.splits = 1;  // capturing, or no memory: the unsplit kernel
    }
    return ojx::launch_gemm_mfma(x, packed, scales, bias, y, part, c, M, N, K, dtype, s, gs, fmt,
                                 bwd);
}

__attribute__((visibility("default"))) int ojx_e8t_gemm_fwd(const void* x, const uint8_t* packed,
                                                            const uint16_t* scales,
                                                            const void* bias, void* y, int64_t M,
                                                            int64_t N, int64_t K, int64_t gs,
                                                            int dtype, void* stream) {
    if (int r = check_gemm_args(x, packed, scales, y, M, N, K, gs, dtype)) return r;
    if (M == 0 || N == 0) return OJX_OK;
    if (int r = check_device()) return r;
    hipStream_t s = (hipStream_t)stream;
    // 4 < M <= 16 on a layer too small for the streaming mask kernel (< 1024 row tiles): one
    // 16-row tile per workgroup, K split over its waves, weights in the B operand
    if (M > 4 && (N + 15) / 16 < 1024 &&
        ojx::gemv2m_supported(x, packed, scales, y, M, N, K, gs, dtype, ojx::kFmtTernary))
        return done(ojx::launch_gemv2m(x, packed, scales, bias, y, M, N, K, gs, dtype, s,
                                       ojx::kFmtTernary),
                    "e8t gemv launch");
    if (K > 0 && ojx::gemv_supported(x, packed, scales, y, M, N, K, gs, dtype)) {
        ojx::GemvLaunch a{};
        ojx::GemvJob& j = a.inl[0];
        j.x = x; j.packed = packed; j.scales = scales; j.bias = bias; j.y = y;
        j.N = N; j.K = K; j.y_col = 0; j.y_ld = N; j.wg_begin = 0;
        a.njobs = 1;
        a.M = (int)M;
        const ojx::GemvPlan plan = ojx::gemv_pick((N + 15) / 16, M);
        return done(ojx::launch_gemv(a, plan, ojx::gemv_wgs_for(N, plan), dtype, s),
                    "e8t gemv launch");
    }
    if (M > 16 && ojx::gemm_mfma_supported(x, packed, scales, M, N, K, gs, dtype))
        return done(launch_mfma(x, packed, scales, bias, y, M, N, K, gs, dtype, s,
                                ojx::kFmtTernary),
                    "e8t gemm_mfma launch");
    return done(ojx::launch_gemm_generic_fwd(x, packed, scales, bias, y, M, N, K, gs, dtype, s),
                "e8t gemm_fwd launch");
}

static_assert(sizeof(ojx_e8t_gemv_job) == sizeof(ojx::GemvJob), "job layout");
static_assert(offsetof(ojx_e8t_gemv_job, wg_begin) == offsetof(ojx::GemvJob, wg_begin),
              "job layout");

static int plan_jobs(ojx_e8t_gemv_job* jobs, int njobs, int64_t M, int dtype, int64_t* grid,
                     ojx::GemvPlan* plan, bool fill) {
    if (njobs <= 0 || !jobs) return fail(OJX_EINVAL, "empty job list");
    if (dtype != OJX_BF16 && dtype != OJX_F16)
        return fail(OJX_EDTYPE, "grouped GEMV takes F16 or BF16 activations (got %d)", dtype);
    if (M < 1 || M > 16) return fail(OJX_ELAYOUT, "grouped GEMV needs 1 <= M <= 16 (got %lld)",
                                     (long long)M);
    int64_t tiles = 0;
    for (int i = 0; i < njobs; ++i) {
        const ojx_e8t_gemv_job& j = jobs[i];
        if (j.N < 1 || j.K < 256 || j.K % 256 != 0)
            return fail(OJX_ELAYOUT, "job %d: needs N >= 1 and K %% 256 == 0 (N=%lld K=%lld)", i,
                        (long long)j.N, (long long)j.K);
        if (!ojx::gemv_shape_ok(j.N, j.K))
            return fail(OJX_ELAYOUT, "job %d: layer too large for 32-bit offsets", i);
        if (!j.packed || !j.scales) return fail(OJX_EINVAL, "job %d: null weight pointer", i);
        if (((uintptr_t)j.packed & 3u) || ((uintptr_t)j.scales & 3u) || ((uintptr_t)j.x & 15u) ||
            ((uintptr_t)j.y & 1u) || ((uintptr_t)j.bias & 1u))
            return fail(OJX_ELAYOUT, "job %d: misaligned pointer", i);
        const int64_t ld = j.y_ld ? j.y_ld : j.N;
        if (j.y_col < 0 || ld < j.y_col + j.N)
            return fail(OJX_ELAYOUT, "job %d: y_ld %lld < y_col %lld + N %lld", i, (long long)ld,
                        (long long)j.y_col, (long long)j.N);
        tiles += (j.N + 15) / 16;
    }
    *plan = ojx::gemv_pick(tiles, M);
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
    return done(ojx::launch_gemv(a, plan, grid, dtype, (hipStream_t)stream),
                "e8t grouped gemv launch");
}

__attribute__((visibility("default"))) int ojx_e8t_gemm_bwd_dx(const void* grad_y,
                                                               const uint8_t* packed,
                                                               const uint16_t* scales,
                                                               void* grad_x, int64_t M, int64_t N,
                                                               int64_t K, int64_t gs, int dtype,
                                                               void* stream) {
    if (int r = check_gemm_args(grad_y, packed, scales, grad_x, M, K, N, gs, dtype)) return r;
    if (M == 0 || K == 0) return OJX_OK;
    if (int r = check_device()) return r;
    hipStream_t s = (hipStream_t)stream;
    if (N > 0 && ojx::gemm_mfma_supported(grad_y, packed, scales, M, N, K, gs, dtype,
                                          ojx::kFmtTernary, true))
        return done(launch_mfma(grad_y, packed, scales, nullptr, grad_x, M, N, K, gs, dtype, s,
                                ojx::kFmtTernary, true),
                    "e8t gemm_mfma bwd launch");
    return done(ojx::launch_gemm_generic_bwd(grad_y, packed, scales, grad_x, M, N, K, gs, dtype, s),
                "e8t gemm_bwd_dx launch");
}

// ------------------------------------------------------------------ 2-bit E8

static int check_gs_multiple(int64_t gs, int64_t unit) {
    if (gs <= 0 || gs % unit != 0)
        return fail(OJX_ELAYOUT, "group_size must be a positive multiple of %lld (got %lld)",
                    (long long)unit, (long long)gs);
    return OJX_OK;
}

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

static int check_gemm2_args(const void* a, const uint8_t* packed, const uint16_t* scales,
                            const void* out, int64_t M, int64_t N, int64_t K, int64_t gs,
                            int dtype) {
    if (M < 0 || N < 0 || K < 0) return fail(OJX_EINVAL, "negative size M=%lld N=%lld K=%lld",
                                             (long long)M, (long long)N, (long long)K);
    if (!valid_dtype(dtype)) return fail(OJX_EDTYPE, "unknown dtype code %d", dtype);
    if (int r = check_gs_multiple(gs, 4)) return r;
    if (M > 0 && N > 0) {
        if (!out) return fail(OJX_EINVAL, "null output pointer");
        if (K > 0 && (!a || !packed || !scales)) return fail(OJX_EINVAL, "null input pointer");
    }
    return OJX_OK;
}

__attribute__((visibility("default"))) int ojx_e8_gemm_fwd(const void* x, const uint8_t* packed,
                                                           const uint16_t* scales,
                                                           const void* bias, void* y, int64_t M,
                                                           int64_t N, int64_t K, int64_t gs,
                                                           int dtype, void* stream) {
    if (int r = check_gemm2_args(x, packed, scales, y, M, N, K, gs, dtype)) return r;
    if (M == 0 || N == 0) return OJX_OK;
    if (int r = check_device()) return r;
    hipStream_t s = (hipStream_t)stream;
    if (ojx::gemv2_supported(x, packed, scales, y, M, N, K, gs, dtype))
        return done(ojx::launch_gemv2(x, packed, scales, bias, y, M, N, K, gs, dtype, s),
                    "e8 gemv launch");
    if (ojx::gemv2m_supported(x, packed, scales, y, M, N, K, gs, dtype, ojx::kFmt2Bit))
        return done(ojx::launch_gemv2m(x, packed, scales, bias, y, M, N, K, gs, dtype, s,
                                       ojx::kFmt2Bit),
                    "e8 gemv launch");
    if (ojx::gemm_mfma_supported(x, packed, scales, M, N, K, gs, dtype, ojx::kFmt2Bit))
        return done(launch_mfma(x, packed, scales, bias, y, M, N, K, gs, dtype, s, ojx::kFmt2Bit),
                    "e8 gemm_mfma launch");
    return done(ojx::launch_gemm_generic_fwd(x, packed, scales, bias, y, M, N, K, gs, dtype, s,
                                             ojx::kFmt2Bit),
                "e8 gemm_fwd launch");
}

__attribute__((visibility("default"))) int ojx_e8_gemm_bwd_dx(const void* grad_y,
                                                              const uint8_t* packed,
                                                              const uint16_t* scales,
                                                              void* grad_x, int64_t M, int64_t N,
                                                              int64_t K, int64_t gs, int dtype,
                                                              void* stream) {
    if (int r = check_gemm2_args(grad_y, packed, scales, grad_x, M, K, N, gs, dtype)) return r;
    if (M == 0 || K == 0) return OJX_OK;
    if (int r = check_device()) return r;
    hipStream_t s = (hipStream_t)stream;
    if (N > 0 && ojx::gemm_mfma_supported(grad_y, packed, scales, M, N, K, gs, dtype,
                                          ojx::kFmt2Bit, true))
        return done(launch_mfma(grad_y, packed, scales, nullptr, grad_x, M, N, K, gs, dtype, s,
                                ojx::kFmt2Bit, true),
                    "e8 gemm_mfma bwd launch");
    return done(ojx::launch_gemm_generic_bwd(grad_y, packed, scales, grad_x, M, N, K, gs, dtype, s,
                                             ojx::kFmt2Bit),
                "e8 gemm_bwd_dx launch");
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

static int check_gemm1_args(const void* a, const uint8_t* codes, const uint16_t* scales,
                            const void* out, int64_t M, int64_t N, int64_t K, int64_t gs,
                            int dtype) {
    if (M < 0 || N < 0 || K < 0) return fail(OJX_EINVAL, "negative size M=%lld N=%lld K=%lld",
                                             (long long)M, (long long)N, (long long)K);
    if (!valid_dtype(dtype)) return fail(OJX_EDTYPE, "unknown dtype code %d", dtype);
    if (int r = check_gs_multiple(gs, 8)) return r;
    if (M > 0 && N > 0) {
        if (!out) return fail(OJX_EINVAL, "null output pointer");
        if (K > 0 && (!a || !codes || !scales)) return fail(OJX_EINVAL, "null input pointer");
    }
    return OJX_OK;
}

__attribute__((visibility("default"))) int ojx_e8r_gemm_fwd(const void* x, const uint8_t* codes,
                                                            const uint16_t* scales,
                                                            const void* bias, void* y, int64_t M,
                                                            int64_t N, int64_t K, int64_t gs,
                                                            int dtype, void* stream) {
    if (int r = check_gemm1_args(x, codes, scales, y, M, N, K, gs, dtype)) return r;
    if (M == 0 || N == 0) return OJX_OK;
    if (int r = check_device()) return r;
    hipStream_t s = (hipStream_t)stream;
    if (ojx::gemv2m_supported(x, codes, scales, y, M, N, K, gs, dtype, ojx::kFmtRoot))
        return done(ojx::launch_gemv2m(x, codes, scales, bias, y, M, N, K, gs, dtype, s,
                                       ojx::kFmtRoot),
                    "e8r gemv launch");
    if (ojx::gemm_mfma_supported(x, codes, scales, M, N, K, gs, dtype, ojx::kFmtRoot))
        return done(launch_mfma(x, codes, scales, bias, y, M, N, K, gs, dtype, s, ojx::kFmtRoot),
                    "e8r gemm_mfma launch");
    return done(ojx::launch_gemm_generic_fwd(x, codes, scales, bias, y, M, N, K, gs, dtype, s,
                                             ojx::kFmtRoot),
                "e8r gemm_fwd launch");
}

__attribute__((visibility("default"))) int ojx_e8r_gemm_bwd_dx(const void* grad_y,
                                                               const uint8_t* codes,
                                                               const uint16_t* scales,
                                                               void* grad_x, int64_t M, int64_t N,
                                                               int64_t K, int64_t gs, int dtype,
                                                               void* stream) {
    if (int r = check_gemm1_args(grad_y, codes, scales, grad_x, M, K, N, gs, dtype)) return r;
    if (M == 0 || K == 0) return OJX_OK;
    if (int r = check_device()) return r;
    hipStream_t s = (hipStream_t)stream;
    if (N > 0 && ojx::gemm_mfma_supported(grad_y, codes, scales, M, N, K, gs, dtype,
                                          ojx::kFmtRoot, true))
        return done(launch_mfma(grad_y, codes, scales, nullptr, grad_x, M, N, K, gs, dtype, s,
                                ojx::kFmtRoot, true),
                    "e8r gemm_mfma bwd launch");
    return done(ojx::launch_gemm_generic_bwd(grad_y, codes, scales, grad_x, M, N, K, gs, dtype, s,
                                             ojx::kFmtRoot),
                "e8r gemm_bwd_dx launch");
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
