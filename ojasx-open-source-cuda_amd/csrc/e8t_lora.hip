// e8t_lora.hip -- down-projection of a LoRA adapter for the fused E8 forwards.
//
// E8LatticeLinear.forward adds scaling * ((x @ A) @ B) to the E8 op's output
// (ojasx2/math/lattice.py:839-842; A [in, r], B [r, out]).  The fused forwards of this
// library add u @ B inside their output epilogue (before the one rounding to the activation
// dtype), with u = scaling * (x @ A) in fp32 [M, r] computed here: one workgroup per
// activation row, the 256 threads splitting K, r partial sums per thread reduced across the
// wave by shuffles and across the waves through LDS.

#include <hip/hip_runtime.h>

#include "e8t_device.h"
#include "e8t_internal.h"

namespace ojx {

constexpr int kLoraThreads = 256;

template <int DT, int RMAX>
__global__ __launch_bounds__(kLoraThreads) void lora_down_kernel(
    const void* __restrict__ x, const void* __restrict__ a, float* __restrict__ u, int64_t K,
    int r, float scaling, int64_t ldu) {
    __shared__ float red[kLoraThreads / 64][RMAX];
    const int64_t m = blockIdx.x;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    float acc[RMAX];
#pragma unroll
    for (int j = 0; j < RMAX; ++j) acc[j] = 0.f;
    for (int64_t k = tid; k < K; k += kLoraThreads) {
        const float xv = load_as_f32<DT>(x, m * K + k);
#pragma unroll
        for (int j = 0; j < RMAX; ++j)
            if (j < r) acc[j] = __builtin_fmaf(xv, load_as_f32<DT>(a, k * r + j), acc[j]);
    }
#pragma unroll
    for (int j = 0; j < RMAX; ++j) {
        float v = acc[j];
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
        acc[j] = v;
    }
    if (lane == 0)
#pragma unroll
        for (int j = 0; j < RMAX; ++j) red[wave][j] = acc[j];
    __syncthreads();
    if (tid < r) {
        float v = 0.f;
#pragma unroll
        for (int w = 0; w < kLoraThreads / 64; ++w) v += red[w][tid];
        u[m * ldu + tid] = scaling * v;
    }
}

template <int DT>
static hipError_t lora_down_dt(const void* x, const void* a, int64_t M, int64_t K, int r,
                               float scaling, float* u, int64_t ldu, hipStream_t s) {
    const dim3 grid((unsigned)M), block(kLoraThreads);
    if (r <= 8) hipLaunchKernelGGL((lora_down_kernel<DT, 8>), grid, block, 0, s, x, a, u, K, r, scaling, ldu);
    else if (r <= 16) hipLaunchKernelGGL((lora_down_kernel<DT, 16>), grid, block, 0, s, x, a, u, K, r, scaling, ldu);
    else if (r <= 32) hipLaunchKernelGGL((lora_down_kernel<DT, 32>), grid, block, 0, s, x, a, u, K, r, scaling, ldu);
    else hipLaunchKernelGGL((lora_down_kernel<DT, 64>), grid, block, 0, s, x, a, u, K, r, scaling, ldu);
    return hipGetLastError();
}

hipError_t launch_lora_down(const void* x, const void* a, int64_t M, int64_t K, int64_t r,
                            float scaling, int dt, float* u, int64_t ldu, hipStream_t stream) {
    if (M <= 0) return hipSuccess;
    if (r < 1 || r > kLoraMaxRank || M > 0x7FFFFFFF) return hipErrorInvalidValue;
    switch (dt) {
        case kF32: return lora_down_dt<kF32>(x, a, M, K, (int)r, scaling, u, ldu, stream);
        case kF16: return lora_down_dt<kF16>(x, a, M, K, (int)r, scaling, u, ldu, stream);
        default: return lora_down_dt<kBF16>(x, a, M, K, (int)r, scaling, u, ldu, stream);
    }
}

}  // namespace ojx
