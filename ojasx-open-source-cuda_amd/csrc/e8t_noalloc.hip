// e8t_noalloc.hip -- the fused ternary forward for callers that cannot allocate device
// memory (code under graph capture that must not grow a memory pool, tight serving loops,
// harnesses that forbid hipMalloc): ojx_e8t_gemm_fwd with the prefill K split's fp32 partial
// sums in a static device array instead of a caller workspace.
//
// The array lives in this file's code object: each GPU the library runs this entry point on
// holds one copy (kScratchBytes) until the process ends.  Host code never uses the array's
// name as an address (on the host it is only a stand-in symbol): the device address of each
// GPU's copy is looked up once per device with hipGetSymbolAddress and kept.
//
// A shape whose planned K split needs more than kScratchBytes is refused.  That is a policy:
// the workspace entry point would run it with the split capped to what fits, but a smaller
// split sums the partials in another order, and this entry point's output is defined as the
// workspace entry point's output with the planned workspace, bit for bit.
//
// Every call on one GPU shares that GPU's copy.  Calls ordered on one stream are safe;
// calls that overlap on one GPU (different streams, or several host threads on different
// streams) race on it.  The split kernels write every partial sum they later read, so the
// array needs no clearing between calls.

#include <hip/hip_runtime.h>

#include <cstdio>
#include <mutex>

#include "../../include/ojasx_e8t.h"
#include "e8t_internal.h"

namespace {

constexpr size_t kScratchBytes = size_t(64) << 20;  // every Llama-3-8B prefill shape fits

__device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_mu;
void* g_scratch_dev[kMaxDevices];  // device address of `scratch` per device; null: not yet

// Address of the current device's copy of `scratch`, looked up on the device's first call.
int scratch_address(void** out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        return ojx::api_fail(OJX_EHIP, "hipGetDevice failed");
    }
    if (dev < 0 || dev >= kMaxDevices) return ojx::api_fail(OJX_EDEVICE, "device index out of range");
    std::lock_guard<std::mutex> lock(g_mu);
    if (!g_scratch_dev[dev]) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) {
            char msg[160];
            snprintf(msg, sizeof msg, "hipGetSymbolAddress(scratch) on device %d: %s", dev,
                     hipGetErrorString(e));
            (void)hipGetLastError();
            return ojx::api_fail(OJX_EHIP, msg);
        }
        g_scratch_dev[dev] = p;
    }
    *out = g_scratch_dev[dev];
    return OJX_OK;
}

}  // namespace

extern "C" __attribute__((visibility("default"))) int ojx_e8t_gemm_fwd_noalloc(
    const void* x, const uint8_t* packed, const uint16_t* scales, const void* bias, void* y,
    int64_t M, int64_t N, int64_t K, int64_t gs, int dtype, void* stream) {
    size_t need = 0;
    if (int r = ojx_gemm_workspace_bytes(OJX_FMT_TERNARY, 0, M, N, K, gs, dtype, &need)) return r;
    if (need > kScratchBytes) {
        char msg[200];
        snprintf(msg, sizeof msg,
                 "M=%lld N=%lld K=%lld needs %zu bytes of K-split scratch; the static scratch "
                 "holds %zu (use ojx_e8t_gemm_fwd with a workspace)",
                 (long long)M, (long long)N, (long long)K, need, kScratchBytes);
        return ojx::api_fail(OJX_ELAYOUT, msg);
    }
    void* ws = nullptr;
    if (int r = scratch_address(&ws)) return r;
    return ojx_e8t_gemm_fwd(x, packed, scales, bias, y, M, N, K, gs, dtype, ws, kScratchBytes,
                            stream);
}
