// e8t_capi.cpp -- extern "C" entry points of libojasx_e8t.so (declared in
// include/ojasx_e8t.h).  Validates arguments the way the reference's native
// binding does (ojasx_math_bindings.cpp:17-34, 414-433), checks the device,
// picks a kernel and enqueues it on the caller's stream.  No allocation, no
// locks on the launch path, no mutable state other than a per-device arch
// cache and a thread-local error message.

#include <hip/hip_runtime.h>

#include <atomic>
#include <cstdarg>
#include <cstdio>
#include <cstring>

#include "../../include/ojasx_e8t.h"
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

__attribute__((visibility("default"))) int ojx_e8t_gemm_fwd(const void* x, const uint8_t* packed,
                                                            const uint16_t* scales,
                                                            const void* bias, void* y, int64_t M,
                                                            int64_t N, int64_t K, int64_t gs,
                                                            int dtype, void* stream) {
    if (int r = check_gemm_args(x, packed, scales, y, M, N, K, gs, dtype)) return r;
    if (M == 0 || N == 0) return OJX_OK;
    if (int r = check_device()) return r;
    hipStream_t s = (hipStream_t)stream;
    return done(ojx::launch_gemm_generic_fwd(x, packed, scales, bias, y, M, N, K, gs, dtype, s),
                "e8t gemm_fwd launch");
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
    return done(ojx::launch_gemm_generic_bwd(grad_y, packed, scales, grad_x, M, N, K, gs, dtype, s),
                "e8t gemm_bwd_dx launch");
}

}  // extern "C"
