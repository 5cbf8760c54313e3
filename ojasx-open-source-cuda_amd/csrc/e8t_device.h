// e8t_device.h -- device helpers shared by the E8 kernels (gfx950): ternary 1.5-bit and
// 2-bit codes.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ojx {

enum : int { kF32 = 0, kF16 = 1, kBF16 = 2, kF64 = 3 /* fwht32 only */ };

// ---------------------------------------------------------------- conversions

__device__ __forceinline__ float f16_bits_to_f32(uint32_t h) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t b) {
    return __uint_as_float(b << 16);
}

// fp32 -> bf16 bits, round-nearest-even, NaN -> 0x7FC0 (torch's c10::BFloat16 rule).
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return 0x7FC0u;
    u += 0x7FFFu + ((u >> 16) & 1u);
    return u >> 16;
}

// fp32 -> bf16 bits, round-nearest-even, by the hardware conversion (v_cvt_pk_bf16_f32):
// one instruction instead of the integer sequence above.  For operands of the kernels' own
// arithmetic (scales, 2-bit and 1-bit value words): finite values round as above, and a
// NaN stays a NaN, whose bits never reach memory (stores go through f32_to_bf16_bits).
__device__ __forceinline__ uint32_t bf16_bits_hw(float f) {
    return (uint32_t)__builtin_bit_cast(uint16_t, (__bf16)f);
}

// fp32 -> fp16 bits, round-nearest-even (v_cvt_f16_f32), subnormals kept.
__device__ __forceinline__ uint32_t f32_to_f16_bits(float f) {
    return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)f);
}

template <int DT> struct Elem;
template <> struct Elem<kF32> { using T = float; };
template <> struct Elem<kF16> { using T = uint16_t; };
template <> struct Elem<kBF16> { using T = uint16_t; };

template <int DT> __device__ __forceinline__ float load_as_f32(const void* p, int64_t i) {
    if constexpr (DT == kF32) return ((const float*)p)[i];
    else if constexpr (DT == kF16) return f16_bits_to_f32(((const uint16_t*)p)[i]);
    else return bf16_bits_to_f32(((const uint16_t*)p)[i]);
}

template <int DT> __device__ __forceinline__ void store_from_f32(void* p, int64_t i, float v) {
    if constexpr (DT == kF32) ((float*)p)[i] = v;
    else if constexpr (DT == kF16) ((uint16_t*)p)[i] = (uint16_t)f32_to_f16_bits(v);
    else ((uint16_t*)p)[i] = (uint16_t)f32_to_bf16_bits(v);
}

// Keeps v a rounded fp32 value in a register.  Left alone, the compiler fuses a product
// that is then narrowed to fp16 into v_fma_mixlo_f16 with a +0 addend, which turns a -0
// product (a negative coefficient times a zero scale) into +0; the reference keeps -0.
__device__ __forceinline__ void keep_f32(float& v) { asm volatile("" : "+v"(v)); }

// Scale value the reference multiplies decoded coordinates by for activations of
// dtype DT (lattice.py:414-418: scales.to(dtype)): fp32 and fp16 keep the fp16
// value exactly, bf16 rounds it to bf16.
template <int DT> __device__ __forceinline__ float scale_for(uint32_t s16) {
    float s = f16_bits_to_f32(s16);
    if constexpr (DT == kBF16) s = bf16_bits_to_f32(bf16_bits_hw(s));
    return s;
}

// ---------------------------------------------------------------- LoRA epilogue

// Low-rank term of a fused forward with a LoRA adapter (E8LatticeLinear.forward,
// lattice.py:839-842: out + scaling * ((x @ A) @ B)): y[m, n] += sum_j u[m, j] * B[j, n], with
// u = scaling * (x @ A) in fp32 [M, r] (row stride ldu) and B the up-projection [r, N] in the
// activation dtype (row stride ldb).  r == 0: no adapter.
struct LoraEp {
    const float* u;
    const void* b;
    int64_t r;
    int64_t ldu;
    int64_t ldb;
};

template <int DT>
__device__ __forceinline__ float lora_term(const float* u, const void* b, int64_t r, int64_t ldu,
                                           int64_t ldb, int64_t m, int64_t n) {
    float s = 0.f;
    for (int64_t j = 0; j < r; ++j)
        s = __builtin_fmaf(u[m * ldu + j], load_as_f32<DT>(b, j * ldb + n), s);
    return s;
}

template <int DT>
__device__ __forceinline__ float lora_term(const LoraEp& l, int64_t m, int64_t n) {
    return l.r > 0 ? lora_term<DT>(l.u, l.b, l.r, l.ldu, l.ldb, m, n) : 0.f;
}

// ---------------------------------------------------------------- packed codes

// 12-bit code t of the packed stream (lattice.py:397-405).
__device__ __forceinline__ uint32_t load_code(const uint8_t* __restrict__ packed, int64_t t) {
    const uint8_t* b = packed + 3 * (t >> 1);
    if (t & 1) return ((uint32_t)b[1] >> 4) | ((uint32_t)b[2] << 4);
    return (uint32_t)b[0] | (((uint32_t)b[1] & 0x0Fu) << 8);
}

// Coordinate i (0..7, in {-1,0,1}) of codeword `code`: base-3 digit i of raw = 2*code.
__device__ __forceinline__ int code_coord(uint32_t code, int i) {
    const uint32_t pow3[8] = {1, 3, 9, 27, 81, 243, 729, 2187};
    return (int)(((2u * code) / pow3[i]) % 3u) - 1;
}

// ---------------------------------------------------------------- 2-bit E8 codes

// Code formats of the packed weight buffers.
enum : int { kFmtTernary = 0, kFmt2Bit = 1, kFmtRoot = 2 };

// 2-bit code f of the flat stream (E8LatticePacker): four per byte, code j of a byte in
// bits [2j, 2j+2) (lattice.py:242-247).
__device__ __forceinline__ uint32_t load_code2(const uint8_t* __restrict__ packed, int64_t f) {
    return ((uint32_t)packed[f >> 2] >> (2 * (f & 3))) & 3u;
}

// Decoded 2-bit weight under the reference's dtype rule (lattice.py:274-276):
// (code - 1.5) * scales.to(dtype), the product computed in fp32 (exact) and rounded once
// to dtype; returned as its fp32 value.
template <int DT> __device__ __forceinline__ float deq2_value(uint32_t code, uint32_t s16) {
    float p = ((float)code - 1.5f) * scale_for<DT>(s16);
    keep_f32(p);
    if constexpr (DT == kF16) return f16_bits_to_f32(f32_to_f16_bits(p));
    else if constexpr (DT == kBF16) return bf16_bits_to_f32(f32_to_bf16_bits(p));
    else return p;
}

// v rounded once to the activation dtype DT (fp16 or bf16), as bits.
template <int DT>
__device__ __forceinline__ uint32_t rnd_bits(float v) {
    keep_f32(v);
    if constexpr (DT == kF16) return f32_to_f16_bits(v);
    else return bf16_bits_hw(v);
}

// Value words {S0, S1} of one 2-bit scale group (fp16 bits s16): the four weights -B, -A,
// +A, +B (A = rnd(0.5 s), B = rnd(1.5 s), s = scales.to(dtype)) as S1 = -B | -A << 16,
// S0 = A | B << 16, so that byte pair 2c, 2c + 1 of v_perm_b32's {S0, S1} is the weight of
// code c (products exact in fp32; -rnd(x) = rnd(-x)).
template <int DT>
__device__ __forceinline__ uint2 values2(uint32_t s16) {
    const float s = scale_for<DT>(s16 & 0xFFFFu);
    const uint32_t a = rnd_bits<DT>(0.5f * s), b = rnd_bits<DT>(1.5f * s);
    return make_uint2(a | (b << 16), (b ^ 0x8000u) | ((a ^ 0x8000u) << 16));
}

}  // namespace ojx
