// e8t_qat.hip -- Conway-Sloane E8 projection and the QAT straight-through quantizer.
//
// conway_sloane_e8_project (ojasx2/math/lattice.py:162-203) as its torch path computes it
// on a GPU tensor: for each 8-vector x, the nearest point of D8 (round half to even; an odd
// coordinate sum moves the first coordinate with the largest rounding error one step
// towards x) and of D8 + 1/2 (the same on x - 1/2, plus 1/2); the closer one by the
// sequential sum of squared differences, D8 on ties.  fp32 or fp64, one lane per vector.
//
// _E8STEFunction.forward (lattice.py:853-865) on fp32 weights: flat, zero padded to a
// multiple of 8; per 8-vector s = torch.norm(w8)/sqrt(8) + 1e-8 (the CPU norm order:
// squares in fmaf lanes, lanes added left to right), out = project(w8 / s) * s.  The
// backward is the identity (straight through) and lives in the Python layer.

#include "e8t_device.h"
#include "e8t_internal.h"

namespace ojx {

template <typename T> __device__ __forceinline__ T rint_even(T v);
template <> __device__ __forceinline__ float rint_even<float>(float v) { return __builtin_rintf(v); }
template <> __device__ __forceinline__ double rint_even<double>(double v) { return __builtin_rint(v); }

template <typename T>
__device__ __forceinline__ void cs_candidate(const T (&x)[8], T shift, T (&out)[8]) {
#pragma clang fp contract(off)
    T f[8], xs[8];
    int sum = 0;
    int worst = 0;
    T werr = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        xs[i] = x[i] - shift;
        f[i] = rint_even<T>(xs[i]);
        sum += (int)f[i];
        const T err = xs[i] - f[i] < 0 ? f[i] - xs[i] : xs[i] - f[i];
        if (i == 0 || err > werr) {
            werr = err;
            worst = i;
        }
    }
    if (sum & 1) {
#pragma unroll
        for (int i = 0; i < 8; ++i)
            if (i == worst) f[i] = f[i] + ((xs[i] - f[i] < 0) ? (T)-1 : (T)1);
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) out[i] = f[i] + shift;
}

template <typename T>
__device__ __forceinline__ void cs_project8(const T (&x)[8], T (&out)[8]) {
#pragma clang fp contract(off)
    T c1[8], c2[8];
    cs_candidate<T>(x, (T)0, c1);
    cs_candidate<T>(x, (T)0.5, c2);
    T d1 = 0, d2 = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const T a = x[i] - c1[i], b = x[i] - c2[i];
        const T a2 = a * a, b2 = b * b;
        d1 = d1 + a2;
        d2 = d2 + b2;
    }
    const bool first = d1 <= d2;
#pragma unroll
    for (int i = 0; i < 8; ++i) out[i] = first ? c1[i] : c2[i];
}

template <typename T>
__global__ __launch_bounds__(256) void cs_project_kernel(const T* __restrict__ x,
                                                         T* __restrict__ out, int64_t nvec) {
    const int64_t b = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (b >= nvec) return;
    T v[8], p[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = x[8 * b + i];
    cs_project8<T>(v, p);
#pragma unroll
    for (int i = 0; i < 8; ++i) out[8 * b + i] = p[i];
}

__global__ __launch_bounds__(256) void ste_quantize_kernel(const float* __restrict__ w,
                                                           int64_t numel,
                                                           float* __restrict__ out) {
#pragma clang fp contract(off)
    const int64_t b = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (8 * b >= numel) return;
    float x[8], v[8], p[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) x[i] = (8 * b + i < numel) ? w[8 * b + i] : 0.f;  // F.pad
    float acc[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[j] = x[j] * x[j];
    float sum = acc[0];
#pragma unroll
    for (int j = 1; j < 8; ++j) sum = sum + acc[j];
    const float root = 2.8284271247461903f;  // fp32(sqrt(8)), as math.sqrt(8) is rounded
    const float s = __builtin_sqrtf(sum) / root + 1e-8f;
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = x[i] / s;
    cs_project8<float>(v, p);
#pragma unroll
    for (int i = 0; i < 8; ++i)
        if (8 * b + i < numel) out[8 * b + i] = p[i] * s;
}

hipError_t launch_cs_project(const void* x, bool f64, int64_t nvec, void* out,
                             hipStream_t stream) {
    const int64_t blocks = (nvec + 255) / 256;
    if (f64)
        hipLaunchKernelGGL(cs_project_kernel<double>, dim3((unsigned)blocks), dim3(256), 0, stream,
                           (const double*)x, (double*)out, nvec);
    else
        hipLaunchKernelGGL(cs_project_kernel<float>, dim3((unsigned)blocks), dim3(256), 0, stream,
                           (const float*)x, (float*)out, nvec);
    return hipGetLastError();
}

hipError_t launch_ste_quantize(const float* w, int64_t numel, float* out, hipStream_t stream) {
    const int64_t nvec = (numel + 7) / 8;
    const int64_t blocks = (nvec + 255) / 256;
    hipLaunchKernelGGL(ste_quantize_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, w, numel,
                       out);
    return hipGetLastError();
}

}  // namespace ojx
