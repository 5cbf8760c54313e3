// e8t_lora.hip -- down-projection of a LoRA adapter for the fused E8 forwards.
//
// E8LatticeLinear.forward adds scaling * ((x @ A) @ B) to the E8 op's output
// (ojasx2/math/lattice.py:839-842; A [in, r], B [r, out]).  The fused forwards of this
// library add u @ B inside their output epilogue (before the one rounding to the activation
// dtype), with u = scaling * (x @ A) in fp32 [M, r] computed here.  The general kernel takes
// any dtype, K and r: one workgroup per activation row, the 256 threads splitting K, r
// partial sums per thread reduced across the wave by shuffles and across the waves in LDS.

#include <hip/hip_runtime.h>

#include "e8t_device.h"
#include "e8t_internal.h"

namespace ojx {

constexpr int kLoraThreads = 256;  // general kernel

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

// Vector form for 16-bit activations, K % 8 == 0 and r % 8 == 0 (16-byte aligned x and A):
// one workgroup per (activation row, adapter); thread t takes the 8 adapter columns
// 8 (t % RS) .. + 7 (RS = r / 8 rounded up to a power of two) of the 8-k chunks t / RS,
// t / RS + 512 / RS, ...: one 16-byte load of x and eight of A per chunk, two chunks in flight
// per iteration, so a decode-sized K (4096: 512 chunks) is one round trip.  Partial sums are
// added across the lanes of equal column slice by shuffles and across the 8 waves in LDS.
constexpr int kLoraVecThreads = 512;

struct LoraDownArgs {
    LoraDown it[kLoraDownItems];
    const void* x;
    int64_t K;
};

template <int DT>
__device__ __forceinline__ void lora_fma8(const uint4& xv, const uint4 (&av)[8], float (&acc)[8]) {
    const uint32_t xw[4] = {xv.x, xv.y, xv.z, xv.w};
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const uint32_t h = (i & 1) ? (xw[i >> 1] >> 16) : (xw[i >> 1] & 0xFFFFu);
        const float xf = DT == kBF16 ? bf16_bits_to_f32(h) : f16_bits_to_f32(h);
        const uint32_t aw[4] = {av[i].x, av[i].y, av[i].z, av[i].w};
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const uint32_t b = (j & 1) ? (aw[j >> 1] >> 16) : (aw[j >> 1] & 0xFFFFu);
            acc[j] = __builtin_fmaf(xf, DT == kBF16 ? bf16_bits_to_f32(b) : f16_bits_to_f32(b),
                                    acc[j]);
        }
    }
}

// RS: column slices of 8 (ranks up to 8 RS; every adapter of the launch has the same RS)
template <int DT, int RS>
__global__ __launch_bounds__(kLoraVecThreads) void lora_down_vec_kernel(LoraDownArgs args) {
    __shared__ float red[kLoraVecThreads / 64][kLoraMaxRank];
    LoraDown it = args.it[0];
#pragma unroll
    for (int i = 1; i < kLoraDownItems; ++i)
        if ((int)blockIdx.y == i) it = args.it[i];
    const int64_t m = blockIdx.x, K = args.K;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int r = (int)it.r;
    const int sl = tid & (RS - 1);
    constexpr int stride = kLoraVecThreads / RS;
    const int64_t nch = K / 8;
    const bool live = 8 * sl < r;
    const uint16_t* xr = static_cast<const uint16_t*>(args.x) + m * K;
    const uint16_t* a = static_cast<const uint16_t*>(it.a) + 8 * sl;
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int64_t c = tid / RS; c < nch; c += 2 * stride) {
        const int64_t c1 = c + stride;
        const bool two = c1 < nch;
        uint4 x0 = make_uint4(0u, 0u, 0u, 0u), x1 = x0, a0[8], a1[8];
        if (live) {
            x0 = *reinterpret_cast<const uint4*>(xr + 8 * c);
#pragma unroll
            for (int i = 0; i < 8; ++i)
                a0[i] = *reinterpret_cast<const uint4*>(a + (8 * c + i) * r);
            if (two) {
                x1 = *reinterpret_cast<const uint4*>(xr + 8 * c1);
#pragma unroll
                for (int i = 0; i < 8; ++i)
                    a1[i] = *reinterpret_cast<const uint4*>(a + (8 * c1 + i) * r);
            }
        }
        if (live) {
            lora_fma8<DT>(x0, a0, acc);
            if (two) lora_fma8<DT>(x1, a1, acc);
        }
    }
    // lanes of equal slice: lane = sl (mod RS)
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        float v = acc[j];
#pragma unroll
        for (int o = 32; o >= RS; o >>= 1) v += __shfl_xor(v, o);
        acc[j] = v;
    }
    if (lane < RS && live)
#pragma unroll
        for (int j = 0; j < 8; ++j) red[wave][8 * lane + j] = acc[j];
    __syncthreads();
    if (tid < r) {
        float v = 0.f;
#pragma unroll
        for (int w = 0; w < kLoraVecThreads / 64; ++w) v += red[w][tid];
        it.u[m * it.ldu + tid] = it.scaling * v;
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

static bool lora_vec_ok(const void* x, const LoraDown& it, int64_t K, int dt) {
    return (dt == kBF16 || dt == kF16) && K % 8 == 0 && it.r % 8 == 0 &&
           ((uintptr_t)x & 15u) == 0 && ((uintptr_t)it.a & 15u) == 0;
}

hipError_t launch_lora_down(const void* x, int64_t M, int64_t K, int dt, const LoraDown* items,
                            int n, hipStream_t stream) {
    if (M <= 0 || n <= 0) return hipSuccess;
    if (M > 0x7FFFFFFF) return hipErrorInvalidValue;
    for (int i = 0; i < n; ++i)
        if (items[i].r < 1 || items[i].r > kLoraMaxRank) return hipErrorInvalidValue;
    LoraDownArgs args{};
    args.x = x;
    args.K = K;
    int k = 0, rs = 0;
    auto flush = [&]() -> hipError_t {
        if (k == 0) return hipSuccess;
        const dim3 grid((unsigned)M, (unsigned)k), block(kLoraVecThreads);
        if (dt == kF16) {
            switch (rs) {
                case 1: hipLaunchKernelGGL((lora_down_vec_kernel<kF16, 1>), grid, block, 0, stream, args); break;
                case 2: hipLaunchKernelGGL((lora_down_vec_kernel<kF16, 2>), grid, block, 0, stream, args); break;
                case 4: hipLaunchKernelGGL((lora_down_vec_kernel<kF16, 4>), grid, block, 0, stream, args); break;
                default: hipLaunchKernelGGL((lora_down_vec_kernel<kF16, 8>), grid, block, 0, stream, args); break;
            }
        } else {
            switch (rs) {
                case 1: hipLaunchKernelGGL((lora_down_vec_kernel<kBF16, 1>), grid, block, 0, stream, args); break;
                case 2: hipLaunchKernelGGL((lora_down_vec_kernel<kBF16, 2>), grid, block, 0, stream, args); break;
                case 4: hipLaunchKernelGGL((lora_down_vec_kernel<kBF16, 4>), grid, block, 0, stream, args); break;
                default: hipLaunchKernelGGL((lora_down_vec_kernel<kBF16, 8>), grid, block, 0, stream, args); break;
            }
        }
        k = 0;
        return hipGetLastError();
    };
    for (int i = 0; i < n; ++i) {
        const LoraDown& it = items[i];
        if (lora_vec_ok(x, it, K, dt)) {
            const int rsi = it.r <= 8 ? 1 : it.r <= 16 ? 2 : it.r <= 32 ? 4 : 8;
            if (k > 0 && rsi != rs)
                if (hipError_t e = flush()) return e;
            rs = rsi;
            args.it[k++] = it;
            if (k == kLoraDownItems)
                if (hipError_t e = flush()) return e;
            continue;
        }
        hipError_t e;
        switch (dt) {
            case kF32: e = lora_down_dt<kF32>(x, it.a, M, K, (int)it.r, it.scaling, it.u, it.ldu, stream); break;
            case kF16: e = lora_down_dt<kF16>(x, it.a, M, K, (int)it.r, it.scaling, it.u, it.ldu, stream); break;
            default: e = lora_down_dt<kBF16>(x, it.a, M, K, (int)it.r, it.scaling, it.u, it.ldu, stream); break;
        }
        if (e != hipSuccess) return e;
    }
    return flush();
}

hipError_t launch_lora_down(const void* x, const void* a, int64_t M, int64_t K, int64_t r,
                            float scaling, int dt, float* u, int64_t ldu, hipStream_t stream) {
    const LoraDown it{a, u, r, ldu, scaling};
    return launch_lora_down(x, M, K, dt, &it, 1, stream);
}

}  // namespace ojx
