// e8t_codec.hip -- E8 encoder and decoder kernels for gfx950: ternary 1.5-bit
// (TernaryE8LatticePacker) and 2-bit (E8LatticePacker, at the end of the file).
//
// Encoder: bit-exact restatement of TernaryE8LatticePacker.pack
// (ojasx2/math/lattice.py:338-384) as one fused pass: each weight is read once
// from HBM (2 B for fp16/bf16) and 0.25 B of codes + scale is written.  The
// reference's device route runs ~25 ATen element-wise kernels with int64
// temporaries for the same work.
//
// One lane per flat group: the reference's scale is torch's CPU norm, whose
// summation order is a sequential FMA chain per lane j over w[j], w[j+8], ...
// (8 fp32 lanes), so a group's norm is inherently serial over its 8-vectors.  One
// lane owning the group computes it once (gs/8 + 7 adds per group) and then runs
// the gs/8 nearest-point searches of its 8-vectors; splitting a group across
// lanes would cost a cross-lane exchange per link of the chain.
//
// Decoder: restatement of TernaryE8LatticePacker.unpack (lattice.py:386-419),
// one lane per code pair (3 bytes -> 16 weights), exact for every dtype.

#include "e8t_device.h"
#include "e8t_internal.h"
#include "e8t_root.h"

namespace ojx {

// Correctly rounded quotient w / s from the group's reciprocal y = RN(1/s), by one
// residual correction (Markstein, "Computation of elementary functions on the IBM RISC
// System/6000 processor", IBM J. Res. Dev. 34(1), 1990): q = RN(w*y), r = w - q*s exact
// by fma, RN(q + r*y) == RN(w/s).  The residual is formed on w*2^48 and s*2^48 and
// multiplied back by y*2^-48 (exact power-of-two scalings), so it stays a normal number
// for every finite w, including subnormal ones.  Checked against true division on
// 1.28e8 weights from realistic, tiny, huge, subnormal and random-exponent groups (0
// mismatches); the kernel's results are compared bit for bit with the CPU oracle.
struct GroupRecip {
    float s, y, bs, ys;  // s, RN(1/s), s*2^48, y*2^-48
    bool exact;          // s not finite: fall back to true division
};

__device__ __forceinline__ GroupRecip group_recip(float s) {
    GroupRecip g;
    g.s = s;
    g.y = 1.0f / s;
    g.bs = s * 0x1p48f;
    g.ys = g.y * 0x1p-48f;
    g.exact = !__builtin_isfinite(s);
    return g;
}

__device__ __forceinline__ float div_rn(float w, const GroupRecip& g) {
#pragma clang fp contract(off)
    const float q = w * g.y;
    const float r = __builtin_fmaf(-q, g.bs, w * 0x1p48f);
    return __builtin_fmaf(r, g.ys, q);
}

// The same quotient without the 2^48 scaling, for weights that came from fp16: every
// nonzero fp16 value is at least 2^-24 in magnitude, so the residual is a normal fp32
// number already (checked against true division for every finite fp16 w over 6,000 scales
// from 2^-40 to 2^42: 0 mismatches).  w = -0 gives +0 here, as in div_rn.
__device__ __forceinline__ float div_rn_f16in(float w, const GroupRecip& g) {
#pragma clang fp contract(off)
    const float q = w * g.y;
    const float r = __builtin_fmaf(-q, g.s, w);
    return __builtin_fmaf(r, g.y, q);
}

// Nearest point of one 8-vector of the group with fp32 scale s, as lattice.py:357-373:
//   v = w / s (correctly rounded)
//   q = clamp(rint(v), -1, 1); alt = q == 0 ? (v >= 0 ? 1 : -1) : 0
//   pen = (alt - v)^2 - (q - v)^2 (three rounded ops, never contracted)
//   odd sum(q): q[first argmin pen] = alt;  code = sum (q_i + 1) 3^i / 2.
// All integer-valued quantities are carried in fp32, where they are exact.  This is the
// literal form, used when the group's scale is not finite (true division).
__device__ __forceinline__ uint32_t quantize8_exact(const float* __restrict__ w, float s) {
#pragma clang fp contract(off)
    const float pow3[8] = {1.f, 3.f, 9.f, 27.f, 81.f, 243.f, 729.f, 2187.f};
    float v[8], q[8];
    float qsum = 0.f;
    float raw = 3280.f;  // sum of 3^i: the "+1" of every digit
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        v[i] = w[i] / s;
        float r = __builtin_rintf(v[i]);
        r = fmaxf(r, -1.f);
        r = fminf(r, 1.f);
        q[i] = r;
        qsum = qsum + r;
        raw = __builtin_fmaf(r, pow3[i], raw);
    }
    float best_pen = 0.f, best_delta = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        float alt = (q[i] == 0.f) ? (v[i] >= 0.f ? 1.f : -1.f) : 0.f;
        float a = alt - v[i];
        float b = q[i] - v[i];
        float a2 = a * a;
        float b2 = b * b;
        float pen = a2 - b2;
        float delta = (alt - q[i]) * pow3[i];
        if (i == 0 || pen < best_pen) {
            best_pen = pen;
            best_delta = delta;
        }
    }
    // sum(q) is an integer in [-8, 8]; odd parity applies the best flip
    int odd = ((int)qsum) & 1;
    raw = odd ? raw + best_delta : raw;
    return ((uint32_t)raw) >> 1;
}

// The same nearest point for a finite scale, in a reduced form with the same results.
// With d = fl(1 - |v|) and t = fl(fl(d * d) - fl(v * v)):
//   * pen == |t| for every finite fp32 v (q == 0 puts both cases' squares in the same two
//     rounded products: alt - v = +-d, q - v = -v; q != 0 swaps them), so the first argmin
//     of pen is the first argmin of |t|;
//   * alt - q == sgn(v) * sgn(t) for every v with |v| < 2^24, where sgn(-0) = +1 (t >= 0
//     exactly when q == 0, and the reference's alt is +1 for v = -0 since -0 >= 0), so the
//     flip adds +-3^i with the sign of (v < 0) XOR t.
// Both identities were checked exhaustively over all 2^32 fp32 bit patterns.  Here
// |v| <= sqrt(gs) * (1 + eps) (the group's norm bounds every weight).  The quotient can be
// -0: the residual division returns +0 for w = -0, but a negative subnormal weight over a
// scale >= 2 rounds to -0, so v's sign is taken by a comparison, not from its sign bit.
// The parity of sum(q) is the parity of the code's base-3 value, since every power of 3
// is odd.  F16IN: the weights came from fp16.
template <bool F16IN>
__device__ __forceinline__ uint32_t quantize8(const float* __restrict__ w, const GroupRecip& g) {
#pragma clang fp contract(off)
    const float pow3[8] = {1.f, 3.f, 9.f, 27.f, 81.f, 243.f, 729.f, 2187.f};
    float raw = 3280.f;  // sum of 3^i: the "+1" of every digit
    float best_t = 0.f, best_v = 0.f, best_p = 0.f;  // t, v and 3^i of the first argmin
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const float v = F16IN ? div_rn_f16in(w[i], g) : div_rn(w[i], g);
        float r = __builtin_rintf(v);
        r = fmaxf(r, -1.f);
        r = fminf(r, 1.f);
        raw = __builtin_fmaf(r, pow3[i], raw);
        const float d = 1.f - fabsf(v);
        const float d2 = d * d;
        const float v2 = v * v;
        const float t = d2 - v2;
        if (i == 0 || fabsf(t) < fabsf(best_t)) {
            best_t = t;
            best_v = v;
            best_p = pow3[i];
        }
    }
    const uint32_t sg = (best_v < 0.f ? 0x80000000u : 0u) ^ (__float_as_uint(best_t) & 0x80000000u);
    const int ri = (int)raw;  // exact: 0 .. 6560
    const int fix = (ri & 1) ? (int)__uint_as_float(__float_as_uint(best_p) | sg) : 0;
    return (uint32_t)(ri + fix) >> 1;
}

// Group scale (lattice.py:355-356) with torch's CPU norm order:
// 8 fmaf lanes, lane j over elements j, j+8, ...; lanes summed left to right;
// correctly rounded sqrt; true division by fp32(sqrt(gs)); + fp32(1e-8).
template <int GS>
__device__ __forceinline__ float group_scale(const float* __restrict__ w, float root) {
#pragma clang fp contract(off)
    float acc[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[j] = w[j] * w[j];
#pragma unroll
    for (int t = 1; t < GS / 8; ++t)
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[j] = __builtin_fmaf(w[8 * t + j], w[8 * t + j], acc[j]);
    float sum = acc[0];
#pragma unroll
    for (int j = 1; j < 8; ++j) sum = sum + acc[j];
    float nrm = __builtin_sqrtf(sum);
    float s = nrm / root;
    return s + 1e-8f;
}

// Two codes -> 3 bytes (lattice.py:379-383).
__device__ __forceinline__ void pack_pair(uint8_t* b, uint32_t c0, uint32_t c1) {
    b[0] = (uint8_t)(c0 & 0xFFu);
    b[1] = (uint8_t)(((c0 >> 8) & 0x0Fu) | ((c1 & 0x0Fu) << 4));
    b[2] = (uint8_t)((c1 >> 4) & 0xFFu);
}

// Eight weights from a 16-byte aligned, in-range address, as fp32.
template <int WDT>
__device__ __forceinline__ void load8_vec(const void* __restrict__ w, int64_t base, float* out) {
    if constexpr (WDT == kF32) {
        const float4* p = reinterpret_cast<const float4*>((const float*)w + base);
        float4 a = p[0], b = p[1];
        out[0] = a.x; out[1] = a.y; out[2] = a.z; out[3] = a.w;
        out[4] = b.x; out[5] = b.y; out[6] = b.z; out[7] = b.w;
    } else {
        uint4 a = *reinterpret_cast<const uint4*>((const uint16_t*)w + base);
        uint32_t u[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            if constexpr (WDT == kF16) {
                out[2 * i] = f16_bits_to_f32(u[i] & 0xFFFFu);
                out[2 * i + 1] = f16_bits_to_f32(u[i] >> 16);
            } else {
                out[2 * i] = bf16_bits_to_f32(u[i] & 0xFFFFu);
                out[2 * i + 1] = bf16_bits_to_f32(u[i] >> 16);
            }
        }
    }
}

template <int WDT>
__device__ __forceinline__ void load8(const void* __restrict__ w, int64_t base, int64_t numel,
                                      bool vec_ok, float* out) {
    if (vec_ok && base + 8 <= numel) {
        if constexpr (WDT == kF32) {
            const float4* p = reinterpret_cast<const float4*>((const float*)w + base);
            float4 a = p[0], b = p[1];
            out[0] = a.x; out[1] = a.y; out[2] = a.z; out[3] = a.w;
            out[4] = b.x; out[5] = b.y; out[6] = b.z; out[7] = b.w;
        } else {
            uint4 a = *reinterpret_cast<const uint4*>((const uint16_t*)w + base);
            uint32_t u[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                if constexpr (WDT == kF16) {
                    out[2 * i] = f16_bits_to_f32(u[i] & 0xFFFFu);
                    out[2 * i + 1] = f16_bits_to_f32(u[i] >> 16);
                } else {
                    out[2 * i] = bf16_bits_to_f32(u[i] & 0xFFFFu);
                    out[2 * i + 1] = bf16_bits_to_f32(u[i] >> 16);
                }
            }
        }
    } else {
#pragma unroll
        for (int i = 0; i < 8; ++i)
            out[i] = (base + i < numel) ? load_as_f32<WDT>(w, base + i) : 0.f;  // F.pad zeros
    }
}

constexpr int kEncThreads = 256;

// GS in {16, 32, 64}: the group stays in registers.
template <int WDT, int GS>
__global__ __launch_bounds__(kEncThreads) void encode_kernel(
    const void* __restrict__ w, int64_t numel, int64_t ngroups, float root, bool vec_ok,
    uint8_t* __restrict__ packed, uint16_t* __restrict__ scales) {
    constexpr int NV = GS / 8;
    constexpr int BYTES = GS * 3 / 16;
    __shared__ uint8_t stage[kEncThreads * BYTES];
    const int64_t g0 = (int64_t)blockIdx.x * kEncThreads;
    const int64_t g = g0 + threadIdx.x;
    if (g < ngroups) {
        float x[GS];
        if (vec_ok && (g + 1) * GS <= numel) {  // the whole group in range: one address
#pragma unroll
            for (int t = 0; t < NV; ++t) load8_vec<WDT>(w, g * GS + 8 * t, x + 8 * t);
        } else {
#pragma unroll
            for (int t = 0; t < NV; ++t) load8<WDT>(w, g * GS + 8 * t, numel, vec_ok, x + 8 * t);
        }
        const float s = group_scale<GS>(x, root);
        const GroupRecip gr = group_recip(s);
        uint8_t* st = stage + threadIdx.x * BYTES;
        if (!gr.exact) {
#pragma unroll
            for (int p = 0; p < NV / 2; ++p)
                pack_pair(st + 3 * p, quantize8<WDT == kF16>(x + 16 * p, gr),
                          quantize8<WDT == kF16>(x + 16 * p + 8, gr));
        } else {
            for (int p = 0; p < NV / 2; ++p)
                pack_pair(st + 3 * p, quantize8_exact(x + 16 * p, s),
                          quantize8_exact(x + 16 * p + 8, s));
        }
        scales[g] = (uint16_t)f32_to_f16_bits(s);
    }
    __syncthreads();
    // coalesced copy-out of the block's packed bytes
    const int64_t ng = (ngroups - g0) < kEncThreads ? (ngroups - g0) : kEncThreads;
    const int nbytes = (int)ng * BYTES;
    uint8_t* dst = packed + g0 * BYTES;
    if ((((uintptr_t)dst) & 3u) == 0) {
        const int nwords = nbytes >> 2;
        const uint32_t* src32 = reinterpret_cast<const uint32_t*>(stage);
        uint32_t* dst32 = reinterpret_cast<uint32_t*>(dst);
        for (int i = threadIdx.x; i < nwords; i += kEncThreads) dst32[i] = src32[i];
        for (int i = (nwords << 2) + threadIdx.x; i < nbytes; i += kEncThreads) dst[i] = stage[i];
    } else {
        for (int i = threadIdx.x; i < nbytes; i += kEncThreads) dst[i] = stage[i];
    }
}

// Any GS (multiple of 16): two passes over the group (norm, then codes); the
// second pass re-reads the group through the caches.
template <int WDT>
__global__ __launch_bounds__(kEncThreads) void encode_kernel_any(
    const void* __restrict__ w, int64_t numel, int64_t ngroups, int64_t gs, float root,
    uint8_t* __restrict__ packed, uint16_t* __restrict__ scales) {
#pragma clang fp contract(off)
    const int64_t g = (int64_t)blockIdx.x * kEncThreads + threadIdx.x;
    if (g >= ngroups) return;
    const int64_t base = g * gs;
    float acc[8];
    for (int t = 0; t < gs / 8; ++t) {
        float x[8];
        load8<WDT>(w, base + 8 * t, numel, false, x);
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[j] = (t == 0) ? x[j] * x[j] : __builtin_fmaf(x[j], x[j], acc[j]);
    }
    float sum = acc[0];
#pragma unroll
    for (int j = 1; j < 8; ++j) sum = sum + acc[j];
    float s = __builtin_sqrtf(sum) / root;
    s = s + 1e-8f;
    uint8_t* dst = packed + base * 3 / 16;
    const GroupRecip gr = group_recip(s);
    for (int p = 0; p < gs / 16; ++p) {
        float x[16];
        load8<WDT>(w, base + 16 * p, numel, false, x);
        load8<WDT>(w, base + 16 * p + 8, numel, false, x + 8);
        if (!gr.exact)
            pack_pair(dst + 3 * p, quantize8<WDT == kF16>(x, gr), quantize8<WDT == kF16>(x + 8, gr));
        else pack_pair(dst + 3 * p, quantize8_exact(x, s), quantize8_exact(x + 8, s));
    }
    scales[g] = (uint16_t)f32_to_f16_bits(s);
}

template <int WDT>
static hipError_t launch_encode_t(const void* w, int64_t numel, int64_t gs, uint8_t* packed,
                                  uint16_t* scales, hipStream_t stream) {
    const int64_t padded = numel + (gs - numel % gs) % gs;
    const int64_t ngroups = padded / gs;
    const float root = (float)__builtin_sqrt((double)gs);
    const int64_t blocks = (ngroups + kEncThreads - 1) / kEncThreads;
    const bool vec_ok = (((uintptr_t)w) & 15u) == 0;
    if (gs == 16)
        hipLaunchKernelGGL((encode_kernel<WDT, 16>), dim3((unsigned)blocks), dim3(kEncThreads), 0,
                           stream, w, numel, ngroups, root, vec_ok, packed, scales);
    else if (gs == 32)
        hipLaunchKernelGGL((encode_kernel<WDT, 32>), dim3((unsigned)blocks), dim3(kEncThreads), 0,
                           stream, w, numel, ngroups, root, vec_ok, packed, scales);
    else if (gs == 64)
        hipLaunchKernelGGL((encode_kernel<WDT, 64>), dim3((unsigned)blocks), dim3(kEncThreads), 0,
                           stream, w, numel, ngroups, root, vec_ok, packed, scales);
    else
        hipLaunchKernelGGL((encode_kernel_any<WDT>), dim3((unsigned)blocks), dim3(kEncThreads), 0,
                           stream, w, numel, ngroups, gs, root, packed, scales);
    return hipGetLastError();
}

hipError_t launch_encode(const void* w, int wdt, int64_t numel, int64_t gs, uint8_t* packed,
                         uint16_t* scales, hipStream_t stream) {
    switch (wdt) {
        case kF32: return launch_encode_t<kF32>(w, numel, gs, packed, scales, stream);
        case kF16: return launch_encode_t<kF16>(w, numel, gs, packed, scales, stream);
        default: return launch_encode_t<kBF16>(w, numel, gs, packed, scales, stream);
    }
}

// ---------------------------------------------------------------- decoder

constexpr int kDecThreads = 256;

template <int ODT>
__global__ __launch_bounds__(kDecThreads) void decode_kernel(
    const uint8_t* __restrict__ packed, const uint16_t* __restrict__ scales, int64_t numel,
    int64_t gs, bool vec_ok, void* __restrict__ out) {
    const int64_t p = (int64_t)blockIdx.x * kDecThreads + threadIdx.x;  // code pair
    const int64_t e0 = p * 16;
    if (e0 >= numel) return;
    const uint32_t b0 = packed[3 * p], b1 = packed[3 * p + 1], b2 = packed[3 * p + 2];
    uint32_t raw0 = 2u * (b0 | ((b1 & 0x0Fu) << 8));
    uint32_t raw1 = 2u * ((b1 >> 4) | (b2 << 4));
    const float s = scale_for<ODT>(scales[e0 / gs]);  // gs % 16 == 0: one group per pair
    float v[16];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        v[i] = (float)((int)(raw0 % 3u) - 1) * s;
        v[8 + i] = (float)((int)(raw1 % 3u) - 1) * s;
        keep_f32(v[i]);  // -1 * 0 stays -0 (see keep_f32)
        keep_f32(v[8 + i]);
        raw0 /= 3u;
        raw1 /= 3u;
    }
    if (vec_ok && e0 + 16 <= numel) {
        if constexpr (ODT == kF32) {
            float4* o = reinterpret_cast<float4*>((float*)out + e0);
#pragma unroll
            for (int i = 0; i < 4; ++i) o[i] = make_float4(v[4 * i], v[4 * i + 1], v[4 * i + 2], v[4 * i + 3]);
        } else {
            uint32_t h[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                uint32_t lo, hi;
                if constexpr (ODT == kF16) { lo = f32_to_f16_bits(v[2 * i]); hi = f32_to_f16_bits(v[2 * i + 1]); }
                else { lo = f32_to_bf16_bits(v[2 * i]); hi = f32_to_bf16_bits(v[2 * i + 1]); }
                h[i] = lo | (hi << 16);
            }
            uint4* o = reinterpret_cast<uint4*>((uint16_t*)out + e0);
            o[0] = make_uint4(h[0], h[1], h[2], h[3]);
            o[1] = make_uint4(h[4], h[5], h[6], h[7]);
        }
    } else {
#pragma unroll
        for (int i = 0; i < 16; ++i)
            if (e0 + i < numel) store_from_f32<ODT>(out, e0 + i, v[i]);
    }
}

hipError_t launch_decode(const uint8_t* packed, const uint16_t* scales, int64_t numel, int64_t gs,
                         int odt, void* out, hipStream_t stream) {
    const int64_t pairs = (numel + 15) / 16;
    const int64_t blocks = (pairs + kDecThreads - 1) / kDecThreads;
    const bool vec_ok = (((uintptr_t)out) & 15u) == 0;
    switch (odt) {
        case kF32:
            hipLaunchKernelGGL((decode_kernel<kF32>), dim3((unsigned)blocks), dim3(kDecThreads), 0,
                               stream, packed, scales, numel, gs, vec_ok, out);
            break;
        case kF16:
            hipLaunchKernelGGL((decode_kernel<kF16>), dim3((unsigned)blocks), dim3(kDecThreads), 0,
                               stream, packed, scales, numel, gs, vec_ok, out);
            break;
        default:
            hipLaunchKernelGGL((decode_kernel<kBF16>), dim3((unsigned)blocks), dim3(kDecThreads), 0,
                               stream, packed, scales, numel, gs, vec_ok, out);
            break;
    }
    return hipGetLastError();
}

// ---------------------------------------------------------------- 2-bit encoder
//
// E8LatticePacker.pack (lattice.py:213-249), bit-exact: the same scale (torch's norm
// order, correctly rounded quotients) and per 8-vector
//   xs = w/s - 0.5; f2 = clamp(rint(xs), -2, 1)
//   alt = xs >= f2 ? clamp(f2 + 1, -2, 1) : clamp(f2 - 1, -2, 1)
//   pen = (alt - xs)^2 - (f2 - xs)^2 (rounded ops, never contracted)
//   odd sum(f2): f2[first argmin pen] = alt;  code_i = f2_i + 2
// A clamped coordinate has alt == f2 and pen 0; as the first minimum its "flip" is a no-op
// and the vector keeps its odd sum, exactly as in the reference.  Returns the 8 codes as
// 16 bits (two packed bytes, code i in bits [2i, 2i+2)).

template <bool EXACT>
__device__ __forceinline__ uint32_t quantize8_2bit(const float* __restrict__ w,
                                                   const GroupRecip& g) {
#pragma clang fp contract(off)
    const float pow4[8] = {1.f, 4.f, 16.f, 64.f, 256.f, 1024.f, 4096.f, 16384.f};
    float xs[8], f2[8];
    float fsum = 0.f;
    float codes = 0.f;  // sum (f2_i + 2) 4^i: exact in fp32
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const float v = EXACT ? w[i] / g.s : div_rn(w[i], g);
        xs[i] = v - 0.5f;
        float r = __builtin_rintf(xs[i]);
        r = fmaxf(r, -2.f);
        r = fminf(r, 1.f);
        f2[i] = r;
        fsum = fsum + r;
        codes = __builtin_fmaf(r + 2.f, pow4[i], codes);
    }
    float best_pen = 0.f, best_delta = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const float up = fminf(f2[i] + 1.f, 1.f), dn = fmaxf(f2[i] - 1.f, -2.f);
        const float alt = xs[i] >= f2[i] ? up : dn;
        const float a = alt - xs[i];
        const float b = f2[i] - xs[i];
        const float a2 = a * a;
        const float b2 = b * b;
        const float pen = a2 - b2;
        const float delta = (alt - f2[i]) * pow4[i];
        if (i == 0 || pen < best_pen) {
            best_pen = pen;
            best_delta = delta;
        }
    }
    const int odd = ((int)fsum) & 1;  // sum(f2) is an integer in [-16, 8]
    codes = odd ? codes + best_delta : codes;
    return (uint32_t)codes;
}

// GS in {8, 16, 32, 64}: the group stays in registers; bytes staged in LDS and written
// coalesced.
template <int WDT, int GS>
__global__ __launch_bounds__(kEncThreads) void encode2_kernel(
    const void* __restrict__ w, int64_t numel, int64_t ngroups, float root, bool vec_ok,
    uint8_t* __restrict__ packed, uint16_t* __restrict__ scales) {
    constexpr int NV = GS / 8;
    constexpr int BYTES = GS / 4;
    __shared__ uint8_t stage[kEncThreads * BYTES];
    const int64_t g0 = (int64_t)blockIdx.x * kEncThreads;
    const int64_t g = g0 + threadIdx.x;
    if (g < ngroups) {
        float x[GS];
        if (vec_ok && (g + 1) * GS <= numel) {  // the whole group in range: one address
#pragma unroll
            for (int t = 0; t < NV; ++t) load8_vec<WDT>(w, g * GS + 8 * t, x + 8 * t);
        } else {
#pragma unroll
            for (int t = 0; t < NV; ++t) load8<WDT>(w, g * GS + 8 * t, numel, vec_ok, x + 8 * t);
        }
        const float s = group_scale<GS>(x, root);
        const GroupRecip gr = group_recip(s);
        uint8_t* st = stage + threadIdx.x * BYTES;
#pragma unroll
        for (int t = 0; t < NV; ++t) {
            const uint32_t c = gr.exact ? quantize8_2bit<true>(x + 8 * t, gr)
                                        : quantize8_2bit<false>(x + 8 * t, gr);
            st[2 * t] = (uint8_t)(c & 0xFFu);
            st[2 * t + 1] = (uint8_t)(c >> 8);
        }
        scales[g] = (uint16_t)f32_to_f16_bits(s);
    }
    __syncthreads();
    const int64_t ng = (ngroups - g0) < kEncThreads ? (ngroups - g0) : kEncThreads;
    const int nbytes = (int)ng * BYTES;
    uint8_t* dst = packed + g0 * BYTES;
    if ((((uintptr_t)dst) & 3u) == 0) {
        const int nwords = nbytes >> 2;
        const uint32_t* src32 = reinterpret_cast<const uint32_t*>(stage);
        uint32_t* dst32 = reinterpret_cast<uint32_t*>(dst);
        for (int i = threadIdx.x; i < nwords; i += kEncThreads) dst32[i] = src32[i];
        for (int i = (nwords << 2) + threadIdx.x; i < nbytes; i += kEncThreads) dst[i] = stage[i];
    } else {
        for (int i = threadIdx.x; i < nbytes; i += kEncThreads) dst[i] = stage[i];
    }
}

// Any GS (multiple of 8): norm pass, then the codes, re-reading the group.
template <int WDT>
__global__ __launch_bounds__(kEncThreads) void encode2_kernel_any(
    const void* __restrict__ w, int64_t numel, int64_t ngroups, int64_t gs, float root,
    uint8_t* __restrict__ packed, uint16_t* __restrict__ scales) {
#pragma clang fp contract(off)
    const int64_t g = (int64_t)blockIdx.x * kEncThreads + threadIdx.x;
    if (g >= ngroups) return;
    const int64_t base = g * gs;
    float acc[8];
    for (int t = 0; t < gs / 8; ++t) {
        float x[8];
        load8<WDT>(w, base + 8 * t, numel, false, x);
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[j] = (t == 0) ? x[j] * x[j] : __builtin_fmaf(x[j], x[j], acc[j]);
    }
    float sum = acc[0];
#pragma unroll
    for (int j = 1; j < 8; ++j) sum = sum + acc[j];
    float s = __builtin_sqrtf(sum) / root;
    s = s + 1e-8f;
    uint8_t* dst = packed + base / 4;
    const GroupRecip gr = group_recip(s);
    for (int t = 0; t < gs / 8; ++t) {
        float x[8];
        load8<WDT>(w, base + 8 * t, numel, false, x);
        const uint32_t c = gr.exact ? quantize8_2bit<true>(x, gr) : quantize8_2bit<false>(x, gr);
        dst[2 * t] = (uint8_t)(c & 0xFFu);
        dst[2 * t + 1] = (uint8_t)(c >> 8);
    }
    scales[g] = (uint16_t)f32_to_f16_bits(s);
}

template <int WDT>
static hipError_t launch_encode2_t(const void* w, int64_t numel, int64_t gs, uint8_t* packed,
                                   uint16_t* scales, hipStream_t stream) {
    const int64_t padded = numel + (gs - numel % gs) % gs;
    const int64_t ngroups = padded / gs;
    const float root = (float)__builtin_sqrt((double)gs);
    const int64_t blocks = (ngroups + kEncThreads - 1) / kEncThreads;
    const bool vec_ok = (((uintptr_t)w) & 15u) == 0;
    switch (gs) {
        case 8:
            hipLaunchKernelGGL((encode2_kernel<WDT, 8>), dim3((unsigned)blocks), dim3(kEncThreads),
                               0, stream, w, numel, ngroups, root, vec_ok, packed, scales);
            break;
        case 16:
            hipLaunchKernelGGL((encode2_kernel<WDT, 16>), dim3((unsigned)blocks),
                               dim3(kEncThreads), 0, stream, w, numel, ngroups, root, vec_ok,
                               packed, scales);
            break;
        case 32:
            hipLaunchKernelGGL((encode2_kernel<WDT, 32>), dim3((unsigned)blocks),
                               dim3(kEncThreads), 0, stream, w, numel, ngroups, root, vec_ok,
                               packed, scales);
            break;
        case 64:
            hipLaunchKernelGGL((encode2_kernel<WDT, 64>), dim3((unsigned)blocks),
                               dim3(kEncThreads), 0, stream, w, numel, ngroups, root, vec_ok,
                               packed, scales);
            break;
        default:
            hipLaunchKernelGGL((encode2_kernel_any<WDT>), dim3((unsigned)blocks),
                               dim3(kEncThreads), 0, stream, w, numel, ngroups, gs, root, packed,
                               scales);
            break;
    }
    return hipGetLastError();
}

hipError_t launch_encode2(const void* w, int wdt, int64_t numel, int64_t gs, uint8_t* packed,
                          uint16_t* scales, hipStream_t stream) {
    switch (wdt) {
        case kF32: return launch_encode2_t<kF32>(w, numel, gs, packed, scales, stream);
        case kF16: return launch_encode2_t<kF16>(w, numel, gs, packed, scales, stream);
        default: return launch_encode2_t<kBF16>(w, numel, gs, packed, scales, stream);
    }
}

// ---------------------------------------------------------------- 2-bit decoder
//
// E8LatticePacker.unpack (lattice.py:252-279): one lane per 16 weights (4 bytes), each
// (code - 1.5) * scales.to(dtype) rounded once to dtype.

template <int ODT>
__global__ __launch_bounds__(kDecThreads) void decode2_kernel(
    const uint8_t* __restrict__ packed, const uint16_t* __restrict__ scales, int64_t numel,
    int64_t padded, int64_t gs, bool vec_ok, void* __restrict__ out) {
    const int64_t p = (int64_t)blockIdx.x * kDecThreads + threadIdx.x;
    const int64_t e0 = p * 16;
    if (e0 >= numel) return;
    uint32_t word;
    if (e0 + 16 <= padded && (((uintptr_t)packed) & 3u) == 0) {
        word = *reinterpret_cast<const uint32_t*>(packed + e0 / 4);
    } else {
        word = 0;
        for (int b = 0; b < 4 && e0 + 4 * b < padded; ++b)
            word |= (uint32_t)packed[e0 / 4 + b] << (8 * b);
    }
    const uint32_t s0 = scales[e0 / gs];  // gs % 8 == 0: each run of 8 is one group
    const uint32_t s1 = (e0 + 8 < padded) ? scales[(e0 + 8) / gs] : s0;
    float v[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) v[i] = deq2_value<ODT>((word >> (2 * i)) & 3u, i < 8 ? s0 : s1);
    if (vec_ok && e0 + 16 <= numel) {
        if constexpr (ODT == kF32) {
            float4* o = reinterpret_cast<float4*>((float*)out + e0);
#pragma unroll
            for (int i = 0; i < 4; ++i) o[i] = make_float4(v[4 * i], v[4 * i + 1], v[4 * i + 2], v[4 * i + 3]);
        } else {
            uint32_t h[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                uint32_t lo, hi;
                if constexpr (ODT == kF16) { lo = f32_to_f16_bits(v[2 * i]); hi = f32_to_f16_bits(v[2 * i + 1]); }
                else { lo = f32_to_bf16_bits(v[2 * i]); hi = f32_to_bf16_bits(v[2 * i + 1]); }
                h[i] = lo | (hi << 16);
            }
            uint4* o = reinterpret_cast<uint4*>((uint16_t*)out + e0);
            o[0] = make_uint4(h[0], h[1], h[2], h[3]);
            o[1] = make_uint4(h[4], h[5], h[6], h[7]);
        }
    } else {
#pragma unroll
        for (int i = 0; i < 16; ++i)
            if (e0 + i < numel) store_from_f32<ODT>(out, e0 + i, v[i]);
    }
}

hipError_t launch_decode2(const uint8_t* packed, const uint16_t* scales, int64_t numel,
                          int64_t gs, int odt, void* out, hipStream_t stream) {
    const int64_t padded = numel + (gs - numel % gs) % gs;
    const int64_t quads = (numel + 15) / 16;
    const int64_t blocks = (quads + kDecThreads - 1) / kDecThreads;
    const bool vec_ok = (((uintptr_t)out) & 15u) == 0;
    switch (odt) {
        case kF32:
            hipLaunchKernelGGL((decode2_kernel<kF32>), dim3((unsigned)blocks), dim3(kDecThreads), 0,
                               stream, packed, scales, numel, padded, gs, vec_ok, out);
            break;
        case kF16:
            hipLaunchKernelGGL((decode2_kernel<kF16>), dim3((unsigned)blocks), dim3(kDecThreads), 0,
                               stream, packed, scales, numel, padded, gs, vec_ok, out);
            break;
        default:
            hipLaunchKernelGGL((decode2_kernel<kBF16>), dim3((unsigned)blocks), dim3(kDecThreads),
                               0, stream, packed, scales, numel, padded, gs, vec_ok, out);
            break;
    }
    return hipGetLastError();
}

// ---------------------------------------------------------------- 1-bit Root-E8 encoder
//
// RootE8LatticePacker.pack (lattice.py:473-509), per flat group of gs weights:
//   s = torch.norm(w)/sqrt(gs) + 1e-8 (the CPU norm order, as the other packers);
//   v = w / s; code = argmax over the 256 table rows u of v . u/|u| (first maximal index);
//   scale = sum(w * q) / max(sum(q * q), 1e-8) for q = table[code], stored as fp16.
// The code search is root_code (e8t_root.h).  Both sums run in torch's CPU order for a
// contiguous last dim: four
// 8-lane accumulators over the 8-blocks of each 32-block, later 8-blocks into the first
// accumulator, accumulators added in order, then the 8 lanes left to right.

// torch's CPU row-sum order (see above), fed one 8-block at a time.
struct TorchRowSum {
    float acc[4][8];
    int block;
    int main_blocks;  // 8-blocks inside whole 32-blocks
    __device__ __forceinline__ void init(int64_t n) {
#pragma unroll
        for (int a = 0; a < 4; ++a)
#pragma unroll
            for (int j = 0; j < 8; ++j) acc[a][j] = 0.f;
        block = 0;
        main_blocks = (int)((n / 8) / 4 * 4);
    }
    __device__ __forceinline__ void add8(const float (&x)[8]) {
#pragma clang fp contract(off)
        const int a = block < main_blocks ? (block & 3) : 0;
#pragma unroll
        for (int q = 0; q < 4; ++q)
            if (q == a)
#pragma unroll
                for (int j = 0; j < 8; ++j) acc[q][j] = acc[q][j] + x[j];
        ++block;
    }
    __device__ __forceinline__ float result() const {
#pragma clang fp contract(off)
        float lane[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) lane[j] = ((acc[0][j] + acc[1][j]) + acc[2][j]) + acc[3][j];
        float s = lane[0];
#pragma unroll
        for (int j = 1; j < 8; ++j) s = s + lane[j];
        return s;
    }
};

// Codes of one group whose weights are read 8 at a time by `get(t, x)`; accumulates the
// MMSE sums; returns the fp16 scale bits.
// NV: the group's 8-blocks when known at compile time (the loop is then unrolled and a
// register-resident group is indexed statically), else 0 and gs / 8 at run time.
template <int NV = 0, typename Get>
__device__ __forceinline__ uint32_t root_group(const Get& get, int64_t gs, float s,
                                               uint8_t* codes_out) {
#pragma clang fp contract(off)
    const GroupRecip gr = group_recip(s);
    TorchRowSum num, den;
    num.init(gs);
    den.init(gs);
    const int64_t nv = NV > 0 ? NV : gs / 8;
#pragma unroll
    for (int64_t t = 0; t < nv; ++t) {
        float x[8], v[8];
        get(t, x);
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = gr.exact ? x[i] / s : div_rn(x[i], gr);
        const uint32_t c = gr.exact ? root_code_full(v) : root_code_fast(v);
        codes_out[t] = (uint8_t)c;
        float wq[8], qq[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float q = (float)kRootTable.c[c][i];
            wq[i] = x[i] * q;
            qq[i] = q * q;
        }
        num.add8(wq);
        den.add8(qq);
    }
    float d = den.result();
    d = d < 1e-8f ? 1e-8f : d;
    return f32_to_f16_bits(num.result() / d);
}

// GS in {8, 16, 32, 64}: the group stays in registers; code bytes staged in LDS and written
// coalesced.
template <int WDT, int GS>
__global__ __launch_bounds__(kEncThreads) void encode1_kernel(
    const void* __restrict__ w, int64_t numel, int64_t ngroups, float root, bool vec_ok,
    uint8_t* __restrict__ codes, uint16_t* __restrict__ scales) {
    constexpr int NV = GS / 8;
    __shared__ uint8_t stage[kEncThreads * NV];
    const int64_t g0 = (int64_t)blockIdx.x * kEncThreads;
    const int64_t g = g0 + threadIdx.x;
    if (g < ngroups) {
        float x[GS];
        if (vec_ok && (g + 1) * GS <= numel) {  // the whole group in range: one address
#pragma unroll
            for (int t = 0; t < NV; ++t) load8_vec<WDT>(w, g * GS + 8 * t, x + 8 * t);
        } else {
#pragma unroll
            for (int t = 0; t < NV; ++t) load8<WDT>(w, g * GS + 8 * t, numel, vec_ok, x + 8 * t);
        }
        const float s = group_scale<GS>(x, root);
        auto get = [&](int64_t t, float (&o)[8]) {
#pragma unroll
            for (int i = 0; i < 8; ++i) o[i] = x[8 * t + i];
        };
        scales[g] = (uint16_t)root_group<NV>(get, GS, s, stage + threadIdx.x * NV);
    }
    __syncthreads();
    const int64_t ng = (ngroups - g0) < kEncThreads ? (ngroups - g0) : kEncThreads;
    const int nbytes = (int)ng * NV;
    uint8_t* dst = codes + g0 * NV;
    if ((((uintptr_t)dst) & 3u) == 0) {
        const int nwords = nbytes >> 2;
        const uint32_t* src32 = reinterpret_cast<const uint32_t*>(stage);
        uint32_t* dst32 = reinterpret_cast<uint32_t*>(dst);
        for (int i = threadIdx.x; i < nwords; i += kEncThreads) dst32[i] = src32[i];
        for (int i = (nwords << 2) + threadIdx.x; i < nbytes; i += kEncThreads) dst[i] = stage[i];
    } else {
        for (int i = threadIdx.x; i < nbytes; i += kEncThreads) dst[i] = stage[i];
    }
}

// Any gs (multiple of 8): norm pass, then the codes, re-reading the group.
template <int WDT>
__global__ __launch_bounds__(kEncThreads) void encode1_kernel_any(
    const void* __restrict__ w, int64_t numel, int64_t ngroups, int64_t gs, float root,
    uint8_t* __restrict__ codes, uint16_t* __restrict__ scales) {
#pragma clang fp contract(off)
    const int64_t g = (int64_t)blockIdx.x * kEncThreads + threadIdx.x;
    if (g >= ngroups) return;
    const int64_t base = g * gs;
    float acc[8];
    for (int t = 0; t < gs / 8; ++t) {
        float x[8];
        load8<WDT>(w, base + 8 * t, numel, false, x);
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[j] = (t == 0) ? x[j] * x[j] : __builtin_fmaf(x[j], x[j], acc[j]);
    }
    float sum = acc[0];
#pragma unroll
    for (int j = 1; j < 8; ++j) sum = sum + acc[j];
    float s = __builtin_sqrtf(sum) / root;
    s = s + 1e-8f;
    auto get = [&](int64_t t, float (&o)[8]) { load8<WDT>(w, base + 8 * t, numel, false, o); };
    scales[g] = (uint16_t)root_group(get, gs, s, codes + base / 8);
}

template <int WDT>
static hipError_t launch_encode1_t(const void* w, int64_t numel, int64_t gs, uint8_t* codes,
                                   uint16_t* scales, hipStream_t stream) {
    const int64_t padded = numel + (gs - numel % gs) % gs;
    const int64_t ngroups = padded / gs;
    const float root = (float)__builtin_sqrt((double)gs);
    const int64_t blocks = (ngroups + kEncThreads - 1) / kEncThreads;
    const bool vec_ok = (((uintptr_t)w) & 15u) == 0;
    switch (gs) {
        case 8:
            hipLaunchKernelGGL((encode1_kernel<WDT, 8>), dim3((unsigned)blocks), dim3(kEncThreads),
                               0, stream, w, numel, ngroups, root, vec_ok, codes, scales);
            break;
        case 16:
            hipLaunchKernelGGL((encode1_kernel<WDT, 16>), dim3((unsigned)blocks),
                               dim3(kEncThreads), 0, stream, w, numel, ngroups, root, vec_ok,
                               codes, scales);
            break;
        case 32:
            hipLaunchKernelGGL((encode1_kernel<WDT, 32>), dim3((unsigned)blocks),
                               dim3(kEncThreads), 0, stream, w, numel, ngroups, root, vec_ok,
                               codes, scales);
            break;
        case 64:
            hipLaunchKernelGGL((encode1_kernel<WDT, 64>), dim3((unsigned)blocks),
                               dim3(kEncThreads), 0, stream, w, numel, ngroups, root, vec_ok,
                               codes, scales);
            break;
        default:
            hipLaunchKernelGGL((encode1_kernel_any<WDT>), dim3((unsigned)blocks),
                               dim3(kEncThreads), 0, stream, w, numel, ngroups, gs, root, codes,
                               scales);
            break;
    }
    return hipGetLastError();
}

hipError_t launch_encode1(const void* w, int wdt, int64_t numel, int64_t gs, uint8_t* codes,
                          uint16_t* scales, hipStream_t stream) {
    switch (wdt) {
        case kF32: return launch_encode1_t<kF32>(w, numel, gs, codes, scales, stream);
        case kF16: return launch_encode1_t<kF16>(w, numel, gs, codes, scales, stream);
        default: return launch_encode1_t<kBF16>(w, numel, gs, codes, scales, stream);
    }
}

// ---------------------------------------------------------------- 1-bit decoder
//
// RootE8LatticePacker.unpack (lattice.py:519-533): one lane per 16 weights (two codes),
// table[code][k] * scales.to(dtype) rounded to dtype (the fp32 product is exact).

template <int ODT>
__global__ __launch_bounds__(kDecThreads) void decode1_kernel(
    const uint8_t* __restrict__ codes, const uint16_t* __restrict__ scales, int64_t numel,
    int64_t padded, int64_t gs, bool vec_ok, void* __restrict__ out) {
    const int64_t p = (int64_t)blockIdx.x * kDecThreads + threadIdx.x;
    const int64_t e0 = p * 16;
    if (e0 >= numel) return;
    const uint32_t c0 = codes[e0 / 8];
    const uint32_t c1 = (e0 + 8 < padded) ? codes[e0 / 8 + 1] : 0u;
    const uint32_t s0 = scales[e0 / gs];
    const uint32_t s1 = (e0 + 8 < padded) ? scales[(e0 + 8) / gs] : s0;
    float v[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const float q = (float)kRootTable.c[i < 8 ? c0 : c1][i & 7];
        float prod = q * scale_for<ODT>(i < 8 ? s0 : s1);
        keep_f32(prod);
        v[i] = prod;
    }
    if (vec_ok && e0 + 16 <= numel) {
        if constexpr (ODT == kF32) {
            float4* o = reinterpret_cast<float4*>((float*)out + e0);
#pragma unroll
            for (int i = 0; i < 4; ++i) o[i] = make_float4(v[4 * i], v[4 * i + 1], v[4 * i + 2], v[4 * i + 3]);
        } else {
            uint32_t h[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                uint32_t lo, hi;
                if constexpr (ODT == kF16) { lo = f32_to_f16_bits(v[2 * i]); hi = f32_to_f16_bits(v[2 * i + 1]); }
                else { lo = f32_to_bf16_bits(v[2 * i]); hi = f32_to_bf16_bits(v[2 * i + 1]); }
                h[i] = lo | (hi << 16);
            }
            uint4* o = reinterpret_cast<uint4*>((uint16_t*)out + e0);
            o[0] = make_uint4(h[0], h[1], h[2], h[3]);
            o[1] = make_uint4(h[4], h[5], h[6], h[7]);
        }
    } else {
#pragma unroll
        for (int i = 0; i < 16; ++i)
            if (e0 + i < numel) store_from_f32<ODT>(out, e0 + i, v[i]);
    }
}

hipError_t launch_decode1(const uint8_t* codes, const uint16_t* scales, int64_t numel,
                          int64_t gs, int odt, void* out, hipStream_t stream) {
    const int64_t padded = numel + (gs - numel % gs) % gs;
    const int64_t pairs = (numel + 15) / 16;
    const int64_t blocks = (pairs + kDecThreads - 1) / kDecThreads;
    const bool vec_ok = (((uintptr_t)out) & 15u) == 0;
    switch (odt) {
        case kF32:
            hipLaunchKernelGGL((decode1_kernel<kF32>), dim3((unsigned)blocks), dim3(kDecThreads), 0,
                               stream, codes, scales, numel, padded, gs, vec_ok, out);
            break;
        case kF16:
            hipLaunchKernelGGL((decode1_kernel<kF16>), dim3((unsigned)blocks), dim3(kDecThreads), 0,
                               stream, codes, scales, numel, padded, gs, vec_ok, out);
            break;
        default:
            hipLaunchKernelGGL((decode1_kernel<kBF16>), dim3((unsigned)blocks), dim3(kDecThreads),
                               0, stream, codes, scales, numel, padded, gs, vec_ok, out);
            break;
    }
    return hipGetLastError();
}

}  // namespace ojx
