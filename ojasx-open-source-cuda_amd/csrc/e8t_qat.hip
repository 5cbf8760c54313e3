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
//
// fp16 / bf16 tensors: the reference runs the same torch expressions in the tensor's own
// dtype, so every elementwise op is computed in fp32 and rounded to the dtype, and a sum
// over the last dim adds fp32 values left to right and rounds once (what torch does on the
// CPU).  The half kernels below round at each of those points: x - 1/2, the parity move
// f +- 1 (and the parity test reads the rounded sum), c + 1/2, x - c and its square, the
// squared distances; for the STE the norm, the division by sqrt(8), + 1e-8 (an fp16 zero
// vector then has s = 0 and NaN outputs, as in the reference), w / s and p * s.

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

// ---- fp16 / bf16 forms (HDT = kF16 or kBF16), values carried in fp32
template <int HDT>
__device__ __forceinline__ float rnd_h(float v) {
    if constexpr (HDT == kBF16) return (float)(__bf16)v;
    else return (float)(_Float16)v;
}
template <int HDT>
__device__ __forceinline__ float h_to_f(uint16_t b) {
    if constexpr (HDT == kBF16) return __uint_as_float((uint32_t)b << 16);
    else return f16_bits_to_f32(b);
}
template <int HDT>
__device__ __forceinline__ uint16_t f_to_h(float v) {  // v holds an exact value of the type
    if constexpr (HDT == kBF16) return __builtin_bit_cast(uint16_t, (__bf16)v);
    else return __builtin_bit_cast(uint16_t, (_Float16)v);
}

template <int HDT>
__device__ __forceinline__ void cs_candidate_h(const float (&x)[8], bool shifted, float (&out)[8]) {
#pragma clang fp contract(off)
    float f[8], xs[8];
    float sum = 0.f;
    int worst = 0;
    float werr = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        xs[i] = shifted ? rnd_h<HDT>(x[i] - 0.5f) : x[i];
        f[i] = __builtin_rintf(xs[i]);
        sum = sum + f[i];
        const float err = rnd_h<HDT>(fabsf(xs[i] - f[i]));
        if (i == 0 || err > werr) {
            werr = err;
            worst = i;
        }
    }
    const long long isum = (long long)rnd_h<HDT>(sum);  // the rounded sum decides the parity
    if (isum & 1) {
#pragma unroll
        for (int i = 0; i < 8; ++i)
            if (i == worst) f[i] = rnd_h<HDT>(f[i] + ((xs[i] - f[i] < 0.f) ? -1.f : 1.f));
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) out[i] = shifted ? rnd_h<HDT>(f[i] + 0.5f) : f[i];
}

template <int HDT>
__device__ __forceinline__ void cs_project8_h(const float (&x)[8], float (&out)[8]) {
#pragma clang fp contract(off)
    float c1[8], c2[8];
    cs_candidate_h<HDT>(x, false, c1);
    cs_candidate_h<HDT>(x, true, c2);
    float d1 = 0.f, d2 = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const float a = rnd_h<HDT>(x[i] - c1[i]), b = rnd_h<HDT>(x[i] - c2[i]);
        d1 = d1 + rnd_h<HDT>(a * a);
        d2 = d2 + rnd_h<HDT>(b * b);
    }
    const bool first = rnd_h<HDT>(d1) <= rnd_h<HDT>(d2);
#pragma unroll
    for (int i = 0; i < 8; ++i) out[i] = first ? c1[i] : c2[i];
}

template <int HDT>
__global__ __launch_bounds__(256) void cs_project_half_kernel(const uint16_t* __restrict__ x,
                                                              uint16_t* __restrict__ out,
                                                              int64_t nvec) {
    const int64_t b = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (b >= nvec) return;
    float v[8], p[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = h_to_f<HDT>(x[8 * b + i]);
    cs_project8_h<HDT>(v, p);
#pragma unroll
    for (int i = 0; i < 8; ++i) out[8 * b + i] = f_to_h<HDT>(p[i]);
}

template <int HDT>
__global__ __launch_bounds__(256) void ste_quantize_half_kernel(const uint16_t* __restrict__ w,
                                                                int64_t numel,
                                                                uint16_t* __restrict__ out) {
#pragma clang fp contract(off)
    const int64_t b = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (8 * b >= numel) return;
    float x[8], v[8], p[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) x[i] = (8 * b + i < numel) ? h_to_f<HDT>(w[8 * b + i]) : 0.f;
    float acc = x[0] * x[0];
#pragma unroll
    for (int i = 1; i < 8; ++i) acc = acc + x[i] * x[i];
    const float root = 2.8284271247461903f;  // fp32(sqrt(8))
    float s = rnd_h<HDT>(rnd_h<HDT>(__builtin_sqrtf(acc)) / root);
    s = rnd_h<HDT>(s + 1e-8f);
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = rnd_h<HDT>(x[i] / s);
    cs_project8_h<HDT>(v, p);
#pragma unroll
    for (int i = 0; i < 8; ++i)
        if (8 * b + i < numel) out[8 * b + i] = f_to_h<HDT>(rnd_h<HDT>(p[i] * s));
}

hipError_t launch_cs_project_dt(const void* x, int dt, int64_t nvec, void* out,
                                hipStream_t stream) {
    const int64_t blocks = (nvec + 255) / 256;
    if (dt == kF16)
        hipLaunchKernelGGL(cs_project_half_kernel<kF16>, dim3((unsigned)blocks), dim3(256), 0,
                           stream, (const uint16_t*)x, (uint16_t*)out, nvec);
    else if (dt == kBF16)
        hipLaunchKernelGGL(cs_project_half_kernel<kBF16>, dim3((unsigned)blocks), dim3(256), 0,
                           stream, (const uint16_t*)x, (uint16_t*)out, nvec);
    else
        return launch_cs_project(x, dt == kF64, nvec, out, stream);
    return hipGetLastError();
}

hipError_t launch_ste_quantize_dt(const void* w, int dt, int64_t numel, void* out,
                                  hipStream_t stream) {
    const int64_t blocks = ((numel + 7) / 8 + 255) / 256;
    if (dt == kF16)
        hipLaunchKernelGGL(ste_quantize_half_kernel<kF16>, dim3((unsigned)blocks), dim3(256), 0,
                           stream, (const uint16_t*)w, numel, (uint16_t*)out);
    else if (dt == kBF16)
        hipLaunchKernelGGL(ste_quantize_half_kernel<kBF16>, dim3((unsigned)blocks), dim3(256), 0,
                           stream, (const uint16_t*)w, numel, (uint16_t*)out);
    else
        return launch_ste_quantize((const float*)w, numel, (float*)out, stream);
    return hipGetLastError();
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
