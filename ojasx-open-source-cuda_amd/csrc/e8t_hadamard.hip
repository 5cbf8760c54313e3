// e8t_hadamard.hip -- normalised 32-point Walsh-Hadamard transform of every 32-element
// block of a row-major tensor (fwht_block32, ojasx2/math/lattice.py:91-102).
//
// The reference evaluates it as five torch stages of butterflies -- distance 1, 2, 4, 8, 16
// inside each 32-block, the sum to the lower index and the difference to the upper -- then
// one multiply by 0.1767766952966369 (1/sqrt(32)).  torch computes each stage of a 16-bit
// tensor in fp32 and rounds the result to the tensor's dtype, and multiplies by the scalar
// cast to the compute type (fp32 for fp32/fp16/bf16 tensors, fp64 for fp64).  This kernel
// performs the same rounded operations in the same order, so its output is bit-identical.
//
// Layout: four lanes per 32-block, eight consecutive elements per lane (one 16-byte load for
// 16-bit types); the distance-1, 2 and 4 stages run in registers, distance 8 and 16 exchange
// with the lanes q ^ 1 and q ^ 2 of the block by shuffles.  Lanes past the last block load
// nothing, take part in the shuffles and store nothing.  HBM-bound: 2 * bytes of the tensor.

#include <hip/hip_runtime.h>

#include "e8t_device.h"
#include "e8t_internal.h"

namespace ojx {

constexpr int kFwhtThreads = 256;

template <int DT> struct FwhtVal { using T = float; };
template <> struct FwhtVal<kF64> { using T = double; };

template <int DT>
__device__ __forceinline__ typename FwhtVal<DT>::T fwht_round(typename FwhtVal<DT>::T v) {
    if constexpr (DT == kBF16) return bf16_bits_to_f32(f32_to_bf16_bits(v));
    else if constexpr (DT == kF16) return f16_bits_to_f32(f32_to_f16_bits(v));
    else return v;
}

template <int DT>
__device__ __forceinline__ void fwht_load(const void* x, int64_t e, typename FwhtVal<DT>::T (&v)[8]) {
    if constexpr (DT == kF64) {
        const double2* p = reinterpret_cast<const double2*>(static_cast<const double*>(x) + e);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const double2 d = p[i];
            v[2 * i] = d.x;
            v[2 * i + 1] = d.y;
        }
    } else if constexpr (DT == kF32) {
        const float4* p = reinterpret_cast<const float4*>(static_cast<const float*>(x) + e);
        const float4 a = p[0], b = p[1];
        v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
        v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    } else {
        const uint4 w = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(x) + e);
        const uint32_t u[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            if constexpr (DT == kBF16) {
                v[2 * i] = bf16_bits_to_f32(u[i] & 0xFFFFu);
                v[2 * i + 1] = bf16_bits_to_f32(u[i] >> 16);
            } else {
                v[2 * i] = f16_bits_to_f32(u[i] & 0xFFFFu);
                v[2 * i + 1] = f16_bits_to_f32(u[i] >> 16);
            }
        }
    }
}

template <int DT>
__device__ __forceinline__ void fwht_store(void* y, int64_t e, const typename FwhtVal<DT>::T (&v)[8]) {
    if constexpr (DT == kF64) {
        double2* p = reinterpret_cast<double2*>(static_cast<double*>(y) + e);
#pragma unroll
        for (int i = 0; i < 4; ++i) p[i] = make_double2(v[2 * i], v[2 * i + 1]);
    } else if constexpr (DT == kF32) {
        float4* p = reinterpret_cast<float4*>(static_cast<float*>(y) + e);
        p[0] = make_float4(v[0], v[1], v[2], v[3]);
        p[1] = make_float4(v[4], v[5], v[6], v[7]);
    } else {
        uint32_t u[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t lo = DT == kBF16 ? f32_to_bf16_bits(v[2 * i]) : f32_to_f16_bits(v[2 * i]);
            const uint32_t hi = DT == kBF16 ? f32_to_bf16_bits(v[2 * i + 1])
                                            : f32_to_f16_bits(v[2 * i + 1]);
            u[i] = (lo & 0xFFFFu) | (hi << 16);
        }
        *reinterpret_cast<uint4*>(static_cast<uint16_t*>(y) + e) = make_uint4(u[0], u[1], u[2], u[3]);
    }
}

template <typename T>
__device__ __forceinline__ T shfl_xor_val(T v, int m) {
    if constexpr (sizeof(T) == 8) {
        const unsigned long long b = __double_as_longlong(v);
        const int lo = __shfl_xor((int)(b & 0xFFFFFFFFull), m);
        const int hi = __shfl_xor((int)(b >> 32), m);
        return __longlong_as_double(((unsigned long long)(uint32_t)hi << 32) | (uint32_t)lo);
    } else {
        return __shfl_xor(v, m);
    }
}

// (x and y may be the same buffer: a wave loads all its blocks before the shuffles, and
// every block is read and written by the same four lanes)
template <int DT>
__global__ __launch_bounds__(kFwhtThreads) void fwht32_kernel(const void* x, void* y,
                                                              int64_t blocks) {
    using T = typename FwhtVal<DT>::T;
    const int64_t t = (int64_t)blockIdx.x * kFwhtThreads + threadIdx.x;
    const int64_t blk = t >> 2;
    const int q = (int)(t & 3);  // this lane's 8-element piece of the block
    const bool live = blk < blocks;
    const int64_t e = blk * 32 + 8 * q;
    T v[8];
    if (live) fwht_load<DT>(x, e, v);
    else
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = T(0);
    // distances 1, 2, 4 inside the piece
#pragma unroll
    for (int d = 1; d <= 4; d *= 2)
#pragma unroll
        for (int i = 0; i < 8; ++i)
            if ((i & d) == 0) {
                const T a = v[i], b = v[i + d];
                v[i] = fwht_round<DT>(a + b);
                v[i + d] = fwht_round<DT>(a - b);
            }
    // distance 8 (pieces q, q ^ 1) and 16 (pieces q, q ^ 2): the lower piece keeps a + b,
    // the upper a - b, with a from the lower piece
#pragma unroll
    for (int m = 1; m <= 2; m *= 2) {
        const bool upper = (q & m) != 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const T p = shfl_xor_val(v[i], m);
            v[i] = upper ? fwht_round<DT>(p - v[i]) : fwht_round<DT>(v[i] + p);
        }
    }
    constexpr T kNorm = T(0.1767766952966369);  // the reference's scalar in the compute type
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = fwht_round<DT>(v[i] * kNorm);
    if (live) fwht_store<DT>(y, e, v);
}

hipError_t launch_fwht32(const void* x, int dt, int64_t blocks, void* y, hipStream_t stream) {
    if (blocks <= 0) return hipSuccess;
    const int64_t threads = blocks * 4;
    const int64_t grid = (threads + kFwhtThreads - 1) / kFwhtThreads;
    if (grid > 0x7FFFFFFF) return hipErrorInvalidValue;
    const dim3 g((unsigned)grid), b(kFwhtThreads);
    switch (dt) {
        case kF64: hipLaunchKernelGGL(fwht32_kernel<kF64>, g, b, 0, stream, x, y, blocks); break;
        case kF32: hipLaunchKernelGGL(fwht32_kernel<kF32>, g, b, 0, stream, x, y, blocks); break;
        case kF16: hipLaunchKernelGGL(fwht32_kernel<kF16>, g, b, 0, stream, x, y, blocks); break;
        case kBF16: hipLaunchKernelGGL(fwht32_kernel<kBF16>, g, b, 0, stream, x, y, blocks); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace ojx
