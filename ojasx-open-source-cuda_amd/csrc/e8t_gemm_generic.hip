// e8t_gemm_generic.hip -- general LDS-tiled SIMT kernels for the fused E8 linear
// (ternary 1.5-bit and 2-bit codes).
//
// These cover every shape and dtype the op accepts (fp32 activations, K not a
// multiple of the MFMA chunk, flat layouts whose groups cross rows, as the
// reference's portable path allows: lattice.py:613-624).  Weights are decoded
// per element from the flat index f = n*K + k straight into LDS, so no dense
// weight ever reaches HBM.  fp32 accumulation; the decoded weight follows the
// reference's dtype rule (coord * scales.to(dtype)).

#include "e8t_device.h"
#include "e8t_internal.h"
#include "e8t_root.h"

namespace ojx {

constexpr int kTile = 64;  // output tile edge
constexpr int kChunk = 32; // contraction chunk

// Weight at flat index f under the reference's dtype rule: ternary coord * scale
// (lattice.py:412-419), or 2-bit (code - 1.5) * scale rounded to dtype (lattice.py:274-276).
template <int FMT, int DT>
__device__ __forceinline__ float deq_flat(const uint8_t* __restrict__ packed,
                                          const uint16_t* __restrict__ scales, int64_t f,
                                          int64_t gs) {
    if constexpr (FMT == kFmt2Bit) return deq2_value<DT>(load_code2(packed, f), scales[f / gs]);
    if constexpr (FMT == kFmtRoot) return deq1_value<DT>(packed[f >> 3], (int)(f & 7), scales[f / gs]);
    const uint32_t code = load_code(packed, f >> 3);
    return (float)code_coord(code, (int)(f & 7)) * scale_for<DT>(scales[f / gs]);
}

// y[M,N] = x[M,K] . W[N,K]^T + bias
template <int FMT, int DT>
__global__ __launch_bounds__(256) void gemm_generic_fwd(
    const void* __restrict__ x, const uint8_t* __restrict__ packed,
    const uint16_t* __restrict__ scales, const void* __restrict__ bias, void* __restrict__ y,
    int64_t M, int64_t N, int64_t K, int64_t gs, LoraEp lora) {
    __shared__ float xs[kChunk][kTile + 4];
    __shared__ float ws[kChunk][kTile + 4];
    const int tid = threadIdx.x;
    const int tm = tid >> 4, tn = tid & 15;
    const int64_t m0 = (int64_t)blockIdx.y * kTile, n0 = (int64_t)blockIdx.x * kTile;
    float acc[4][4] = {};
    for (int64_t k0 = 0; k0 < K; k0 += kChunk) {
#pragma unroll
        for (int r = 0; r < (kTile * kChunk) / 256; ++r) {
            const int idx = tid + r * 256;
            const int row = idx / kChunk, kk = idx % kChunk;
            const int64_t gk = k0 + kk;
            const int64_t gm = m0 + row, gn = n0 + row;
            xs[kk][row] = (gm < M && gk < K) ? load_as_f32<DT>(x, gm * K + gk) : 0.f;
            ws[kk][row] = (gn < N && gk < K) ? deq_flat<FMT, DT>(packed, scales, gn * K + gk, gs) : 0.f;
        }
        __syncthreads();
#pragma unroll 8
        for (int kk = 0; kk < kChunk; ++kk) {
            const float4 a = *reinterpret_cast<const float4*>(&xs[kk][tm * 4]);
            const float4 b = *reinterpret_cast<const float4*>(&ws[kk][tn * 4]);
            const float av[4] = {a.x, a.y, a.z, a.w}, bv[4] = {b.x, b.y, b.z, b.w};
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[i][j] = __builtin_fmaf(av[i], bv[j], acc[i][j]);
        }
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int64_t gm = m0 + tm * 4 + i;
        if (gm >= M) continue;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int64_t gn = n0 + tn * 4 + j;
            if (gn >= N) continue;
            float v = acc[i][j];
            if (bias) v += load_as_f32<DT>(bias, gn);
            v += lora_term<DT>(lora, gm, gn);
            store_from_f32<DT>(y, gm * N + gn, v);
        }
    }
}

// gx[M,K] = gy[M,N] . W[N,K]
template <int FMT, int DT>
__global__ __launch_bounds__(256) void gemm_generic_bwd(
    const void* __restrict__ gy, const uint8_t* __restrict__ packed,
    const uint16_t* __restrict__ scales, void* __restrict__ gx, int64_t M, int64_t N, int64_t K,
    int64_t gs) {
    __shared__ float gs_tile[kChunk][kTile + 4];  // [n][m]
    __shared__ float ws[kChunk][kTile + 4];       // [n][k]
    const int tid = threadIdx.x;
    const int tm = tid >> 4, tk = tid & 15;
    const int64_t m0 = (int64_t)blockIdx.y * kTile, k0 = (int64_t)blockIdx.x * kTile;
    float acc[4][4] = {};
    for (int64_t n0 = 0; n0 < N; n0 += kChunk) {
#pragma unroll
        for (int r = 0; r < (kTile * kChunk) / 256; ++r) {
            const int idx = tid + r * 256;
            // gy tile: consecutive threads walk n (contiguous in gy rows)
            {
                const int row = idx / kChunk, nn = idx % kChunk;
                const int64_t gm = m0 + row, gn = n0 + nn;
                gs_tile[nn][row] = (gm < M && gn < N) ? load_as_f32<DT>(gy, gm * N + gn) : 0.f;
            }
            // W tile: consecutive threads walk k (contiguous in a packed row)
            {
                const int nn = idx / kTile, kk = idx % kTile;
                const int64_t gn = n0 + nn, gk = k0 + kk;
                ws[nn][kk] = (gn < N && gk < K) ? deq_flat<FMT, DT>(packed, scales, gn * K + gk, gs) : 0.f;
            }
        }
        __syncthreads();
#pragma unroll 8
        for (int nn = 0; nn < kChunk; ++nn) {
            const float4 a = *reinterpret_cast<const float4*>(&gs_tile[nn][tm * 4]);
            const float4 b = *reinterpret_cast<const float4*>(&ws[nn][tk * 4]);
            const float av[4] = {a.x, a.y, a.z, a.w}, bv[4] = {b.x, b.y, b.z, b.w};
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[i][j] = __builtin_fmaf(av[i], bv[j], acc[i][j]);
        }
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int64_t gm = m0 + tm * 4 + i;
        if (gm >= M) continue;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int64_t gk = k0 + tk * 4 + j;
            if (gk < K) store_from_f32<DT>(gx, gm * K + gk, acc[i][j]);
        }
    }
}

template <int FMT, int DT>
static hipError_t fwd_t(const void* x, const uint8_t* packed, const uint16_t* scales,
                        const void* bias, void* y, int64_t M, int64_t N, int64_t K, int64_t gs,
                        hipStream_t stream, const LoraEp& lora) {
    dim3 grid((unsigned)((N + kTile - 1) / kTile), (unsigned)((M + kTile - 1) / kTile));
    hipLaunchKernelGGL((gemm_generic_fwd<FMT, DT>), grid, dim3(256), 0, stream, x, packed, scales,
                       bias, y, M, N, K, gs, lora);
    return hipGetLastError();
}

template <int FMT, int DT>
static hipError_t bwd_t(const void* gy, const uint8_t* packed, const uint16_t* scales, void* gx,
                        int64_t M, int64_t N, int64_t K, int64_t gs, hipStream_t stream) {
    dim3 grid((unsigned)((K + kTile - 1) / kTile), (unsigned)((M + kTile - 1) / kTile));
    hipLaunchKernelGGL((gemm_generic_bwd<FMT, DT>), grid, dim3(256), 0, stream, gy, packed, scales,
                       gx, M, N, K, gs);
    return hipGetLastError();
}

template <int FMT>
static hipError_t fwd_fmt(const void* x, const uint8_t* packed, const uint16_t* scales,
                          const void* bias, void* y, int64_t M, int64_t N, int64_t K, int64_t gs,
                          int dt, hipStream_t stream, const LoraEp& lora) {
    switch (dt) {
        case kF32: return fwd_t<FMT, kF32>(x, packed, scales, bias, y, M, N, K, gs, stream, lora);
        case kF16: return fwd_t<FMT, kF16>(x, packed, scales, bias, y, M, N, K, gs, stream, lora);
        default: return fwd_t<FMT, kBF16>(x, packed, scales, bias, y, M, N, K, gs, stream, lora);
    }
}

template <int FMT>
static hipError_t bwd_fmt(const void* gy, const uint8_t* packed, const uint16_t* scales, void* gx,
                          int64_t M, int64_t N, int64_t K, int64_t gs, int dt,
                          hipStream_t stream) {
    switch (dt) {
        case kF32: return bwd_t<FMT, kF32>(gy, packed, scales, gx, M, N, K, gs, stream);
        case kF16: return bwd_t<FMT, kF16>(gy, packed, scales, gx, M, N, K, gs, stream);
        default: return bwd_t<FMT, kBF16>(gy, packed, scales, gx, M, N, K, gs, stream);
    }
}

hipError_t launch_gemm_generic_fwd(const void* x, const uint8_t* packed, const uint16_t* scales,
                                   const void* bias, void* y, int64_t M, int64_t N, int64_t K,
                                   int64_t gs, int dt, hipStream_t stream, int fmt,
                                   const LoraEp& lora) {
    if (fmt == kFmtRoot)
        return fwd_fmt<kFmtRoot>(x, packed, scales, bias, y, M, N, K, gs, dt, stream, lora);
    return fmt == kFmt2Bit
               ? fwd_fmt<kFmt2Bit>(x, packed, scales, bias, y, M, N, K, gs, dt, stream, lora)
               : fwd_fmt<kFmtTernary>(x, packed, scales, bias, y, M, N, K, gs, dt, stream, lora);
}

hipError_t launch_gemm_generic_bwd(const void* gy, const uint8_t* packed, const uint16_t* scales,
                                   void* gx, int64_t M, int64_t N, int64_t K, int64_t gs, int dt,
                                   hipStream_t stream, int fmt) {
    if (fmt == kFmtRoot) return bwd_fmt<kFmtRoot>(gy, packed, scales, gx, M, N, K, gs, dt, stream);
    return fmt == kFmt2Bit
               ? bwd_fmt<kFmt2Bit>(gy, packed, scales, gx, M, N, K, gs, dt, stream)
               : bwd_fmt<kFmtTernary>(gy, packed, scales, gx, M, N, K, gs, dt, stream);
}

}  // namespace ojx
