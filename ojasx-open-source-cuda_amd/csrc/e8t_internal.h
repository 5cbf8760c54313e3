// e8t_internal.h -- launchers shared between the kernel files and the C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ojx {

hipError_t launch_encode(const void* w, int wdt, int64_t numel, int64_t gs, uint8_t* packed,
                         uint16_t* scales, hipStream_t stream);

hipError_t launch_decode(const uint8_t* packed, const uint16_t* scales, int64_t numel, int64_t gs,
                         int odt, void* out, hipStream_t stream);

// General tiled kernels: any M, N, K >= 1 (flat layout), any dtype.
hipError_t launch_gemm_generic_fwd(const void* x, const uint8_t* packed, const uint16_t* scales,
                                   const void* bias, void* y, int64_t M, int64_t N, int64_t K,
                                   int64_t gs, int dt, hipStream_t stream);
hipError_t launch_gemm_generic_bwd(const void* gy, const uint8_t* packed, const uint16_t* scales,
                                   void* gx, int64_t M, int64_t N, int64_t K, int64_t gs, int dt,
                                   hipStream_t stream);

}  // namespace ojx
